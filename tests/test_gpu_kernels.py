"""Every kernel against the CPU oracle on random shapes and seeds and at the edges, through the
C ABI (x0ne_core.ops.Kernels): the counterpart of x0ne-core/oracle/tests/gpu_kernels.rs.

Tolerances are the reference's (common/mod.rs:98-107): a bf16 result within 2^-7 of the
oracle, an f32 accumulation within 1e-5 of the sum of its terms' magnitudes, an attention
within 2^-7 of the largest V, a rotation within 1e-3 of the largest value. What a kernel copies
is compared bit for bit, and so are KV-slot indexing (a sentinel-filled paged cache keeps every
byte but the written rows) and the argmax."""
import numpy as np
import pytest

from common import (ATTENTION_ATOL_OF_VMAX, BF16_ATOL, BF16_RTOL, F32_RTOL, ROPE_ATOL_OF_XMAX, O, assert_close,
                    bf16_bits, bf16_vals, bf16s_with_edges, bits_f32, max_abs)

pytestmark = pytest.mark.gpu


def H(q, kv):
    from x0ne_core.ops import Heads
    return Heads(q, kv)


def test_probe_and_launch_checks(kernels):
    """The build path end to end (probe.cu) and the launch argument check (gpu.rs:317-333)."""
    from x0ne_core import Arena, Arg, Class, GpuError
    a = Arena()
    s = a.alloc("out", 1000 * 4, Class.CLIENT_DATA)
    a.freeze(kernels.gpu)
    kernels.gpu.launch("x0ne_probe_iota_u32", 4, 256, [Arg.ptr(a.ptr(s)), Arg.u32(1000)])
    kernels.gpu.sync()
    assert (a.read_array(s, 0, 1000, np.uint32) == np.arange(1000)).all()
    with pytest.raises(GpuError, match="argument 1"):
        kernels.gpu.launch("x0ne_probe_iota_u32", 4, 256, [Arg.ptr(a.ptr(s)), Arg.f32(1.0)])
    with pytest.raises(GpuError):
        kernels.gpu.launch("x0ne_probe_iota_u32", 4, 256, [Arg.ptr(a.ptr(s))])
    with pytest.raises(GpuError):
        kernels.gpu.launch("x0ne_no_such_kernel", 1, 64, [])
    print("MEASURE", kernels.gpu.describe())


def test_the_hardware_bf16_rounding_is_the_references_on_every_f32(kernels):
    """The kernels round with v_cvt_pk_bf16_f32. On the device it is compared with the rounding
    stated on the bits for all 2^32 f32 values; on the host, with the oracle's encoder
    (bf16.rs:11-20), over ranges holding zeros, denormals, ties around 1, the largest finite
    values, infinities and NaNs of both signs."""
    step = 1 << 28
    for base in range(0, 1 << 32, step):
        differ, _ = kernels.probe_bf16_round(base, step)
        assert differ == 0, f"{differ} values from {base:#010x} round differently"
    for base in [0x00000000, 0x007F8000, 0x3F7F8000, 0x3F800000, 0x7F7F0000, 0x7FBF8000, 0x80000000, 0xFF7F0000,
                 0xFFBF8000, 0xFFFF0000]:
        n = 1 << 16
        _, bits = kernels.probe_bf16_round(base, n, read=True)
        vals = (np.arange(n, dtype=np.uint64) + base).astype(np.uint32).view(np.float32)
        want = O.bf16_bits(vals)
        bad = np.flatnonzero(bits != want)
        assert bad.size == 0, f"{base + int(bad[0]):#010x}: {int(bits[bad[0]]):#06x} vs {int(want[bad[0]]):#06x}"


def test_embedding_copies_the_row_bit_for_bit_and_zeroes_a_token_outside(kernels):
    rng = O.Rng(1)
    for hidden in [8, 16, 64, 1024, 4096]:
        for vocab in [1, 2, 7, 300]:
            raw = np.array([rng.next_u64() & 0xFFFF for _ in range(vocab * hidden)], np.uint16)
            table = bf16_vals(raw)
            for token in [0, vocab - 1, rng.below(vocab), vocab, vocab + 1, 0xFFFFFFFF]:
                got = kernels.embedding(raw, hidden, token)
                want = bf16_bits(O.embedding(table, hidden, token))
                # NaN payloads are copied as they are: compare bits of the copy with the table's.
                if token < vocab:
                    assert (got == raw[token * hidden:(token + 1) * hidden]).all(), (hidden, vocab, token)
                else:
                    assert (got == want).all() and (got == 0).all(), (hidden, vocab, token)
    from x0ne_core import FormatError
    for hidden in [0, 4, 12]:
        with pytest.raises(FormatError):
            kernels.embedding(np.zeros(24, np.uint16), hidden, 0)


@pytest.mark.parametrize("seed", range(30))
def test_add_rmsnorm_is_the_oracle_on_random_rows(kernels, seed):
    rng = O.Rng(100 + seed)
    h = rng.pick([1, 2, 7, 8, 64, 255, 256, 257, 1024, 4096, 5120])
    scale = rng.pick([1e-3, 1.0, 30.0, 1e4])
    residual = rng.f32s(h, scale)
    x = bf16s_with_edges(rng, h, scale)
    w = rng.bf16s(h, 2.0)
    eps = rng.pick([1e-6, 1e-5])
    r, out = kernels.add_rmsnorm(residual, bf16_bits(x), bf16_bits(w), eps)
    want_r, want = O.add_rmsnorm(residual, x, w, eps)
    assert (bits_f32(r) == bits_f32(want_r)).all(), "the residual is one f32 addition per value"
    assert_close(f"add_rmsnorm seed {seed} h {h}", bf16_vals(out), want, BF16_ATOL, BF16_RTOL + F32_RTOL)
    # Computed in f64 like the oracle: the bf16 values are the oracle's rounded, but for a value
    # whose f64 lies on a rounding boundary.
    same = (out == bf16_bits(want)).mean()
    print(f"MEASURE add_rmsnorm seed {seed}: {same:.6f} of the values bit-equal to the rounded oracle")


@pytest.mark.parametrize("h", [8, 256, 1024, 4096, 5120, 8192, 9000])
def test_panel_norm_is_the_row_norm_bit_for_bit(kernels, h):
    """The batched step's norm (several rows, out in panels) gives each row the bits of
    x0ne_add_rmsnorm_bf16, past the values a thread keeps in registers too (h > 8192)."""
    rng = O.Rng(130 + h)
    n = 19
    residual = np.stack([rng.f32s(h, 3.0) for _ in range(n)])
    x = np.stack([bf16_bits(bf16s_with_edges(rng, h, 3.0)) for _ in range(n)])
    w = bf16_bits(rng.bf16s(h, 2.0))
    r, out = kernels.add_rmsnorm_panel(residual, x, w, 1e-6)
    for t in range(n):
        r1, o1 = kernels.add_rmsnorm(residual[t], x[t], w, 1e-6)
        assert (bits_f32(r[t]) == bits_f32(r1)).all() and (out[t] == o1).all(), f"h {h} row {t}"


def test_add_rmsnorm_on_zero_denormal_and_non_finite_rows(kernels):
    h = 64
    w = np.ones(h, np.float32)
    def run(residual, x):
        r, out = kernels.add_rmsnorm(residual, bf16_bits(x), bf16_bits(w), 1e-6)
        want_r, want = O.add_rmsnorm(residual, x, w, 1e-6)
        canon = lambda v: np.where(np.isnan(v), np.float32(np.nan), v).view(np.uint32)
        assert (canon(r) == canon(want_r)).all()
        return bf16_vals(out), want
    got, want = run(np.zeros(h, np.float32), np.zeros(h, np.float32))
    assert (got == want).all(), "a zero row stays zero"
    tiny = bf16_vals(np.full(h, 1, np.uint16))
    got, want = run(np.zeros(h, np.float32), tiny)
    assert_close("denormal row", got, want, 1e-30, BF16_RTOL + F32_RTOL)
    for special in [np.nan, np.inf, -np.inf]:
        x = np.ones(h, np.float32)
        x[17] = special
        got, want = run(np.full(h, 0.5, np.float32), x)
        assert (np.isnan(got) == np.isnan(want)).all(), special
        fin = ~np.isnan(want)
        assert (np.abs(got[fin] - want[fin]) <= 1e-6).all(), special


@pytest.mark.parametrize("seed", range(20))
def test_qk_norm_rope_is_the_oracle_and_writes_one_paged_slot(kernels, seed):
    from x0ne_core.ops import CacheAt, inv_freq
    rng = O.Rng(200 + seed)
    kv = rng.pick([1, 2, 4, 8])
    h = H(kv * rng.pick([1, 2, 4]), kv)
    layers = rng.range(1, 3)
    max_ctx = rng.pick([1, 2, 17, 64, 513])
    pos = rng.pick([0, max_ctx - 1, rng.below(max_ctx)])
    at = CacheAt(layers, max_ctx, rng.below(layers), pos)
    theta = rng.pick([1e4, 1e6])
    qkv = bf16s_with_edges(rng, h.q_dim + 2 * h.kv_dim, 8.0)
    qn, kn = rng.bf16s(128, 2.0), rng.bf16s(128, 2.0)
    # Shuffled pages in a pool larger than the sequence needs.
    pages = (max_ctx + 15) // 16
    pool = pages + 3
    page_of = [int(p) for p in np.random.default_rng(seed).permutation(pool)[:pages]]
    out = kernels.qk_norm_rope_kv_write(bf16_bits(qkv), bf16_bits(qn), bf16_bits(kn), h, theta, 1e-6, at,
                                        page_of=page_of, pool=pool)
    q, k, v = O.qk_norm_rope(qkv, qn, kn, inv_freq(128, theta), h.q_heads, h.kv_heads, 128, pos, 1e-6)
    what = f"seed {seed} {h} {at}"
    assert out.rest_untouched, f"{what}: a cache byte outside the slot was written"
    assert (out.v_row == bf16_bits(v)).all(), f"{what}: v is copied"
    for name, got, want in [("q", out.q, q), ("k", out.k_row, k)]:
        assert_close(f"{what} {name}", bf16_vals(got), want, ROPE_ATOL_OF_XMAX * max_abs(want) + BF16_ATOL, BF16_RTOL)
    # The prefill pass's kernel, cos and sin from the RoPE table: the same bits and the same slot.
    rows = kernels.qk_norm_rope_kv_write(bf16_bits(qkv), bf16_bits(qn), bf16_bits(kn), h, theta, 1e-6, at,
                                         page_of=page_of, pool=pool, table=True)
    assert rows.rest_untouched, f"{what} (table): a cache byte outside the slot was written"
    for name, got, want in [("q", rows.q, out.q), ("k", rows.k_row, out.k_row), ("v", rows.v_row, out.v_row)]:
        assert (got == want).all(), f"{what} (table): {name} differs from the direct kernel's"


def test_rope_far_into_a_long_context(kernels):
    """The angle is an f32 product, here as on the device (gpu_kernels.rs:263-292)."""
    from x0ne_core.ops import CacheAt, inv_freq
    h = H(2, 1)
    rng = O.Rng(299)
    qkv = rng.bf16s(h.q_dim + 2 * h.kv_dim, 4.0)
    ones = np.ones(128, np.float32)
    for pos in [4095, 32767, 131071]:
        out = kernels.qk_norm_rope_kv_write(bf16_bits(qkv), bf16_bits(ones), bf16_bits(ones), h, 1e6, 1e-6,
                                            CacheAt(1, pos + 1, 0, pos))
        q, _, _ = O.qk_norm_rope(qkv, ones, ones, inv_freq(128, 1e6), 2, 1, 128, pos, 1e-6)
        assert_close(f"rope at {pos}", bf16_vals(out.q), q, ROPE_ATOL_OF_XMAX * max_abs(q), BF16_RTOL)
        assert out.rest_untouched
        rows = kernels.qk_norm_rope_kv_write(bf16_bits(qkv), bf16_bits(ones), bf16_bits(ones), h, 1e6, 1e-6,
                                             CacheAt(1, pos + 1, 0, pos), table=True)
        assert (rows.q == out.q).all() and (rows.k_row == out.k_row).all(), f"table rope at {pos}"


def test_rope_table_is_the_cosine_and_sine_of_the_f32_angle(kernels):
    """The fused attention's table: for each position and pair, cos and sin in f64 of the f32
    product p * inv_freq[i], within 2 ulp of numpy's (the rotation kernels' own functions give
    the table's bits: the fused-vs-two-kernel test compares the K rows they write bit for bit)."""
    from x0ne_core.ops import inv_freq
    n = 4096
    t = kernels.rope_table(128, 1e6, n)
    inv = inv_freq(128, 1e6)
    angle = (np.arange(n, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float64)
    assert angle.dtype == np.float64 and np.all(angle[1] == inv.astype(np.float64))
    for k, f in [(0, np.cos), (1, np.sin)]:
        want = f(angle)
        err = np.abs(t[:, :, k] - want)
        assert (err <= 2 * np.spacing(np.maximum(np.abs(want), 1e-300))).all(), f"{f.__name__}: {err.max()}"
    assert (t[0, :, 0] == 1.0).all() and (t[0, :, 1] == 0.0).all()


def assert_gemv(what, got, want, magnitude, rounded):
    bound = F32_RTOL * magnitude + (BF16_RTOL * np.abs(want).astype(np.float64) + BF16_ATOL if rounded else 1e-30)
    r = np.abs(got.astype(np.float64) - want.astype(np.float64)) / bound
    print(f"MEASURE {what}: worst ratio {r.max():.4f}")
    assert (r <= 1.0).all(), f"{what}: row {int(np.argmax(r))}"


@pytest.mark.parametrize("seed", range(30))
def test_gemv_is_the_oracle_on_random_shapes(kernels, seed):
    rng = O.Rng(300 + seed)
    rows = rng.pick([1, 2, 3, 8, 127, 1024, 2049])
    cols = rng.pick([1, 2, 8, 9, 64, 1000, 1024, 4096, 12288])
    scale = rng.pick([1e-2, 1.0, 50.0])
    w = bf16s_with_edges(rng, rows * cols, scale)
    x = bf16s_with_edges(rng, cols, scale)
    want = O.gemv(w, rows, cols, x)
    mag = O.gemv_magnitude(w, rows, cols, x)
    what = f"gemv seed {seed} {rows}x{cols}"
    f = kernels.gemv_f32_out(bf16_bits(w), rows, cols, bf16_bits(x))
    assert_gemv(f"{what} f32", f, want, mag, False)
    b = kernels.gemv_bf16_out(bf16_bits(w), rows, cols, bf16_bits(x))
    assert_gemv(f"{what} bf16", bf16_vals(b), want, mag, True)
    # One accumulation, two stores: the bf16 output is the f32 output rounded.
    assert (b == bf16_bits(f)).all(), what


@pytest.mark.parametrize("seed", range(16))
def test_gemm_is_the_oracle_gemv_of_every_row(kernels, seed):
    """Gpu::gemm over many rows (the few-row matrix-core kernel up to 64 rows, this library's
    tiled matrix-core GEMM past them when W's rows are a multiple of 4, a GEMV per row of X
    otherwise): every row of Y is the oracle's GEMV of that row of X within the GEMV tolerance
    (gpu_kernels.rs:331-393), at tile edges of both sides and K tails. The bf16 output is the f32
    output rounded where the same kernel serves both (one accumulation, two stores); the per-row
    GEMV may differ between the two, and, as the reference does for its GEMV
    (gpu_kernels.rs:372-377), the test only reports whether they agree there."""
    rng = O.Rng(700 + seed)
    n = rng.pick([2, 3, 4, 5, 16, 17, 31, 33, 64, 65, 128, 129, 257])
    rows = rng.pick([1, 15, 128, 129, 384, 1000])
    cols = rng.pick([8, 64, 72, 1000, 4096])
    scale = rng.pick([1e-2, 1.0, 50.0])
    w = bf16s_with_edges(rng, rows * cols, scale)
    x = bf16s_with_edges(rng, n * cols, scale)
    f = kernels.gemm(bf16_bits(w), rows, cols, bf16_bits(x), n, True)
    b = kernels.gemm(bf16_bits(w), rows, cols, bf16_bits(x), n, False)
    what = f"gemm seed {seed} {n}x{rows}x{cols}"
    for r in range(n):
        xr = x[r * cols:(r + 1) * cols]
        want = O.gemv(w, rows, cols, xr)
        mag = O.gemv_magnitude(w, rows, cols, xr)
        assert_gemv(f"{what} row {r} f32", f[r], want, mag, False)
        assert_gemv(f"{what} row {r} bf16", bf16_vals(b[r]), want, mag, True)
    same = bool((b == bf16_bits(f).reshape(b.shape)).all())
    if n <= 64 or rows % 4 == 0:
        assert same, what
    else:
        print(f"MEASURE {what}: bf16 out is the rounded f32 out: {same}")
    # Each shape runs the same kernels on every call: the same bits.
    assert (kernels.gemm(bf16_bits(w), rows, cols, bf16_bits(x), n, True).view(np.uint32) == f.view(np.uint32)).all(), what


TILES = {"256x256": 1, "256x128": 2, "128x128": 3}
W_PANELS, X_PANELS = 1, 2


@pytest.mark.parametrize("tile", sorted(TILES))
@pytest.mark.parametrize("seed", range(6))
def test_the_tiled_gemm_is_the_oracle_gemv_at_every_tile(kernels, tile, seed):
    """The prefill passes' GEMM (x0ne_gpu_gemm_tiled) at each of its block tiles, on shapes that
    cut the tiles on every side: tokens from one to past a 256-row tile, W rows a multiple of 4
    that end inside a tile, K tails inside a 32-column fragment (cols a multiple of 8 only) and
    values at the bf16 edges. Every row of Y is the oracle's GEMV of that row of X within the
    GEMV tolerance (gpu_kernels.rs:331-393), the bf16 output is the f32 output rounded (one
    accumulation, two stores), a second call gives the same bits, and W and/or X handed over in
    16-row panels (W rows then a multiple of 16) give the same bits as row-major: the loads fill
    the same fragments, the products sum in the same order."""
    rng = O.Rng(900 + 17 * seed + TILES[tile])
    n = rng.pick([1, 2, 17, 65, 128, 129, 255, 256, 257, 300])
    rows = rng.pick([4, 16, 60, 128, 132, 256, 260, 272, 516, 528])
    cols = rng.pick([8, 24, 32, 40, 96, 1000])
    scale = rng.pick([1e-2, 1.0, 50.0])
    w = bf16s_with_edges(rng, rows * cols, scale)
    x = bf16s_with_edges(rng, n * cols, scale)
    t = TILES[tile]
    f = kernels.gemm(bf16_bits(w), rows, cols, bf16_bits(x), n, True, tile=t)
    b = kernels.gemm(bf16_bits(w), rows, cols, bf16_bits(x), n, False, tile=t)
    what = f"tiled gemm {tile} seed {seed}: {n} tokens x {rows} rows x {cols}"
    for r in range(n):
        xr = x[r * cols:(r + 1) * cols]
        want = O.gemv(w, rows, cols, xr)
        mag = O.gemv_magnitude(w, rows, cols, xr)
        assert_gemv(f"{what} token {r} f32", f[r], want, mag, False)
    assert (b == bf16_bits(f).reshape(b.shape)).all(), f"{what}: bf16 out is the rounded f32 out"
    again = kernels.gemm(bf16_bits(w), rows, cols, bf16_bits(x), n, True, tile=t)
    assert (again.view(np.uint32) == f.view(np.uint32)).all(), f"{what}: the same bits twice"
    for layout in [X_PANELS] + ([W_PANELS, W_PANELS | X_PANELS] if rows % 16 == 0 else []):
        p = kernels.gemm(bf16_bits(w), rows, cols, bf16_bits(x), n, True, tile=t, layout=layout)
        assert (p.view(np.uint32) == f.view(np.uint32)).all(), f"{what}: layout {layout} is row-major's bits"
        pb = kernels.gemm(bf16_bits(w), rows, cols, bf16_bits(x), n, False, tile=t, layout=layout)
        assert (pb == b).all(), f"{what}: layout {layout} bf16"


@pytest.mark.parametrize("name,rows,cols", [("qkv", 6144, 4096), ("o", 4096, 4096), ("gate_up", 24576, 4096),
                                            ("down", 4096, 12288)])
def test_the_tiled_gemm_at_the_prefill_shapes(kernels, name, rows, cols):
    """Qwen3-8B's four projections as a 2048-row prefill pass runs them, the tile the library
    picks for each (x0ne_gpu_gemv past 64 rows), on 300 tokens (two token tiles of every
    shape, the second cut): N(0, 0.02) weights, x of unit scale, against float64 products
    (the oracle's GEMV arithmetic) within the GEMV tolerance; the engine's form (W and X in
    panels, the same tile) gives the same bits."""
    rng = np.random.default_rng(rows + cols)
    n = 300
    w = O.bf16_round(rng.normal(0, 0.02, rows * cols).astype(np.float32))
    x = O.bf16_round(rng.normal(0, 1.0, n * cols).astype(np.float32))
    f = kernels.gemm(bf16_bits(w), rows, cols, bf16_bits(x), n, True)
    W = w.reshape(rows, cols).astype(np.float64)
    X = x.reshape(n, cols).astype(np.float64)
    want = X @ W.T
    mag = np.abs(X) @ np.abs(W).T
    r = np.abs(f.astype(np.float64) - want) / (1e-5 * mag + 1e-30)
    print(f"MEASURE tiled gemm {name} {n}x{rows}x{cols}: worst ratio {r.max():.4f}")
    assert (r <= 1.0).all(), name
    p = kernels.gemm(bf16_bits(w), rows, cols, bf16_bits(x), n, True, tile=0, layout=W_PANELS | X_PANELS)
    assert (p.view(np.uint32) == f.view(np.uint32)).all(), f"{name}: panels"


@pytest.mark.parametrize("seed", range(24))
def test_few_row_gemm_is_the_oracle_and_its_swiglu_the_swiglu_kernel(kernels, seed):
    """The batched step's projection kernel (2 to 64 rows of X, each W row read once) at every
    block size it runs with: every row of Y is the oracle's GEMV within the GEMV tolerance, the
    bf16 output is the f32 output rounded, and the fused SwiGLU (mode 2) over a packed
    [gate; up] W gives the bits of the SwiGLU kernel applied to the bf16 projection (the same
    products in the same order), which is the oracle's SwiGLU of the rounded gate and up."""
    rng = O.Rng(800 + seed)
    n = rng.pick([1, 2, 7, 16, 17, 32, 33, 64])
    rows = rng.pick([1, 16, 17, 100, 256, 1000])
    cols = rng.pick([8, 32, 40, 200, 1024, 4096])
    block = rng.pick([256, 512])
    tt = 1 if n <= 16 else 2 if n <= 32 else 4
    rg = rng.pick([g for (t, g) in kernels.FEW_KERNELS if t == tt])
    rg_glu = rng.pick([g for (t, g) in kernels.FEW_SWIGLU if t == tt])
    scale = rng.pick([1e-2, 1.0, 20.0])
    w = bf16s_with_edges(rng, 2 * rows * cols, scale)
    x = bf16s_with_edges(rng, n * cols, scale)
    what = f"few-row gemm seed {seed} {n}x{rows}x{cols} block {block} row groups {rg}/{rg_glu}"
    f = kernels.gemm_few(bf16_bits(w[:rows * cols]), rows, cols, bf16_bits(x), n, 1, block, rg)
    b = kernels.gemm_few(bf16_bits(w[:rows * cols]), rows, cols, bf16_bits(x), n, 0, block, rg)
    for r in range(n):
        xr = x[r * cols:(r + 1) * cols]
        want = O.gemv(w[:rows * cols], rows, cols, xr)
        mag = O.gemv_magnitude(w[:rows * cols], rows, cols, xr)
        assert_gemv(f"{what} row {r} f32", f[r], want, mag, False)
    assert (b == bf16_bits(f).reshape(b.shape)).all(), f"{what}: bf16 is the f32 rounded"
    gu = kernels.gemm_few(bf16_bits(w), 2 * rows, cols, bf16_bits(x), n, 0, block, rg_glu)
    act = kernels.gemm_few(bf16_bits(w), rows, cols, bf16_bits(x), n, 2, block, rg_glu)
    for r in range(n):
        assert (act[r] == kernels.swiglu(gu[r])).all(), f"{what} row {r}: fused SwiGLU"
        assert_close(f"{what} row {r} swiglu", bf16_vals(act[r]), O.swiglu(bf16_vals(gu[r])), BF16_ATOL, BF16_RTOL)
    # The panel layouts move the same values: the same bits.
    fp = kernels.gemm_few(bf16_bits(w[:rows * cols]), rows, cols, bf16_bits(x), n, 1, block, rg, x_panel=True)
    assert (fp.view(np.uint32) == f.view(np.uint32)).all(), f"{what}: X in panels"
    if rows % 8 == 0:
        ap = kernels.gemm_few(bf16_bits(w), rows, cols, bf16_bits(x), n, 2, block, rg_glu, x_panel=True, y_panel=True)
        assert (ap == act).all(), f"{what}: SwiGLU with X and Y in panels"


@pytest.mark.parametrize("seed", range(12))
def test_few_row_gemm_reads_w_in_panels_bit_for_bit(kernels, seed):
    """W in 16-row panels (FEW_W_PANEL, the batched engine's copy) moves the same values into the
    same products in the same order: Y is bit-equal to the row-major W's, for the f32, bf16 and
    SwiGLU outputs, with X and Y in panels or not, at K tails and every block size."""
    rng = O.Rng(900 + seed)
    n = rng.pick([1, 2, 7, 16, 17, 32, 33, 64])
    rows = rng.pick([16, 32, 48, 256, 1024])
    cols = rng.pick([8, 40, 200, 1024, 4096])
    block = rng.pick([256, 512])
    tt = 1 if n <= 16 else 2 if n <= 32 else 4
    rg = rng.pick([g for (t, g) in kernels.FEW_KERNELS if t == tt])
    rg_glu = rng.pick([g for (t, g) in kernels.FEW_SWIGLU if t == tt])
    xp = rng.pick([False, True])
    w = bf16_bits(bf16s_with_edges(rng, 2 * rows * cols, 1.0))
    x = bf16_bits(bf16s_with_edges(rng, n * cols, 1.0))
    what = f"W panel seed {seed} {n}x{rows}x{cols} block {block} row groups {rg}/{rg_glu} X panel {xp}"
    for mode in (0, 1):
        want = kernels.gemm_few(w[:rows * cols], rows, cols, x, n, mode, block, rg, x_panel=xp)
        got = kernels.gemm_few(w[:rows * cols], rows, cols, x, n, mode, block, rg, x_panel=xp, w_panel=True)
        assert (np.asarray(got).view(np.uint16) == np.asarray(want).view(np.uint16)).all(), f"{what} mode {mode}"
    want = kernels.gemm_few(w, rows, cols, x, n, 2, block, rg_glu, x_panel=xp, y_panel=xp)
    got = kernels.gemm_few(w, rows, cols, x, n, 2, block, rg_glu, x_panel=xp, y_panel=xp, w_panel=True)
    assert (got == want).all(), f"{what}: SwiGLU"
    from x0ne_core import FormatError
    with pytest.raises(FormatError):
        kernels.gemm_few(w[:(rows + 8) * 8], rows + 8, 8, x[:n * 8], n, 0, w_panel=True)


@pytest.mark.parametrize("seed", range(10))
def test_balanced_few_row_gemm_is_the_oracle_and_the_same_bits_every_time(kernels, seed):
    """The balanced few-row kernel (one block per equal run of the groups' steps; groups cut
    between two runs finished by the last block to count): every row of Y is the oracle's GEMV
    within the GEMV tolerance, bf16 Y is f32 Y rounded, a row alone gets the bits it gets in the
    batch, repeated launches give the same bits and leave every count at zero. Runs shorter and
    longer than a group, cut groups, K tails, 4 and 8 wavefronts."""
    rng = O.Rng(1900 + seed)
    n = rng.pick([1, 5, 8, 16])
    rows = 16 * rng.pick([3, 17, 40, 300])
    cols = rng.pick([264, 1024, 2056, 8192])
    block = rng.pick([256, 512])
    groups, steps = rows // 16, -(-cols // 32)
    T = rng.pick([max(block // 64, steps // 2 + 3), steps + 5, 2 * steps - 1, -(-groups * steps // 7)])
    T = max(block // 64, min(T, 4 * steps + 1))
    scale = rng.pick([1e-2, 1.0])
    w = bf16s_with_edges(rng, rows * cols, scale)
    x = bf16s_with_edges(rng, n * cols, scale)
    what = f"balanced few-row seed {seed} {n}x{rows}x{cols} block {block} run {T}"
    f, zero = kernels.gemm_few_bal(bf16_bits(w), rows, cols, bf16_bits(x), n, 1, block, T, calls=2)
    assert zero, f"{what}: counts left at zero"
    for r in range(n):
        xr = x[r * cols:(r + 1) * cols]
        assert_gemv(f"{what} row {r} f32", f[r], O.gemv(w, rows, cols, xr), O.gemv_magnitude(w, rows, cols, xr), False)
    b, _ = kernels.gemm_few_bal(bf16_bits(w), rows, cols, bf16_bits(x), n, 0, block, T)
    assert (b == bf16_bits(f).reshape(b.shape)).all(), f"{what}: bf16 is the f32 rounded"
    f2, _ = kernels.gemm_few_bal(bf16_bits(w), rows, cols, bf16_bits(x), n, 1, block, T)
    assert (f2.view(np.uint32) == f.view(np.uint32)).all(), f"{what}: the same bits again"
    f1, _ = kernels.gemm_few_bal(bf16_bits(w), rows, cols, bf16_bits(x[:cols]), 1, 1, block, T)
    assert (f1[0].view(np.uint32) == f[0].view(np.uint32)).all(), f"{what}: row 0 alone"


@pytest.mark.parametrize("seed", range(16))
def test_the_f64_gemm_is_the_exact_sum_of_the_products(kernels, seed):
    """The exact mode's projection (x0ne_gemm_f64_t*_bf16, and x0ne_gemm_f64_q*_bf16 for up to
    32 rows of X): each output is the f64 sum of its exact bf16 products, rounded to f32 (and the
    bf16 output that f32 rounded). Against the exactly rounded sum (math.fsum): equal in f32 but
    where the f64 sums' own rounding (at most cols x 2^-53 of the sum of the magnitudes) reaches
    an f32 rounding boundary. Every tile width and quad count, K cut into slices (more slices than
    steps too), K tails, rows and tokens past a tile's edge, zeros and denormals among the values."""
    import math
    rng = O.Rng(2000 + seed)
    n = rng.pick([1, 5, 16, 17, 20, 33, 70] if seed < 8 else [1, 3, 4, 5, 8, 13, 20, 31, 32])
    rows = rng.pick([1, 16, 63, 200])
    cols = rng.pick([8, 40, 264, 1032])
    ks = rng.pick([1, 1, 3, 16])
    if seed < 8:
        tt, tq = rng.pick([1, 2, 4]), 0
    else:
        tt, tq = 0, rng.pick([q for q in range(1, 9) if 4 * q >= n])
    scale = rng.pick([1e-2, 1.0])
    w = bf16s_with_edges(rng, rows * cols, scale)
    x = bf16s_with_edges(rng, n * cols, scale)
    what = f"f64 gemm seed {seed} {n}x{rows}x{cols} tiles {tt} quads {tq} K slices {ks}"
    f = kernels.gemm_f64(bf16_bits(w), rows, cols, bf16_bits(x), n, True, tt, ks, tq)
    b = kernels.gemm_f64(bf16_bits(w), rows, cols, bf16_bits(x), n, False, tt, ks, tq)
    assert (b == bf16_bits(f).reshape(b.shape)).all(), f"{what}: bf16 is the f32 rounded"
    W = w.astype(np.float64).reshape(rows, cols)
    X = x.astype(np.float64).reshape(n, cols)
    equal = 0
    for t in range(n):
        for r in range(rows):
            p = X[t] * W[r]
            exact = math.fsum(p)
            got = float(f[t, r])
            want = float(np.float32(exact))
            if got == want or (got != got and want != want):
                equal += 1
                continue
            bound = cols * 2.0 ** -53 * float(np.abs(p).sum())
            assert abs(got - exact) <= abs(want - exact) + bound + np.spacing(np.float32(abs(exact))), \
                f"{what}: token {t} row {r}: {got!r} against {want!r}"
    assert equal >= 0.999 * n * rows, f"{what}: {equal} of {n * rows} equal"


@pytest.mark.parametrize("rows,cols", [(16, 8), (48, 40), (32, 1000), (1024, 4096), (17, 8), (16, 12)])
def test_panel_copy_is_the_panel_layout(kernels, rows, cols):
    """x0ne_panel_bf16 (the load-time copy of a batched engine's weights) writes the host's panel
    layout of the matrix; a shape it does not take (rows not a multiple of 16, cols not of 8)
    leaves the destination untouched."""
    m = O.Rng(rows * 7 + cols).bf16s(rows * cols, 1.0)
    got = kernels.panel(bf16_bits(m), rows, cols)
    if rows % 16 or cols % 8:
        assert (got == 0xFFFF).all()
        return
    from x0ne_core.ops import from_panels, to_panels
    want = to_panels(bf16_bits(m).reshape(rows, cols))
    assert (got == want).all()
    assert (from_panels(got, rows, cols).reshape(-1) == bf16_bits(m)).all()


def test_gemv_carries_non_finite_values_to_the_rows_that_read_them(kernels):
    rows, cols = 16, 64
    rng = O.Rng(399)
    w = rng.bf16s(rows * cols, 1.0)
    for r in range(8):
        w[r * cols + 5] = 0.0
    x = rng.bf16s(cols, 1.0)
    x[5] = np.inf
    got = kernels.gemv_f32_out(bf16_bits(w), rows, cols, bf16_bits(x))
    want = O.gemv(w, rows, cols, x)
    assert (np.isfinite(got) == np.isfinite(want)).all()
    assert (np.isnan(got) == np.isnan(want)).all()


GEOMETRIES = [(1, 1), (2, 1), (4, 2), (16, 8), (32, 8), (40, 8), (64, 8)]
CTXS = [1, 2, 3, 15, 16, 17, 63, 64, 65, 127, 128, 129, 255, 257, 511, 513, 1000, 2048, 4097]


def attention_inputs(rng, ctx, h, scale):
    return (rng.bf16s(h.q_dim, scale), rng.bf16s(ctx * h.kv_dim, scale), bf16s_with_edges(rng, ctx * h.kv_dim, 4.0))


@pytest.mark.parametrize("qh,kvh", GEOMETRIES)
def test_decode_attention_is_the_oracle_around_every_boundary(kernels, qh, kvh):
    """Per-head, split-K with each merge and P in {1, 4, 16, the plan's}, over shuffled pages,
    against the oracle at contexts around the page (16), the tile (64) and larger."""
    h = H(qh, kvh)
    plan = kernels.split_plan(h)
    print(f"MEASURE {qh}/{kvh} heads: P {plan.splits} grouped {plan.grouped} per CU {plan.per_cu}")
    rng = O.Rng(400 + qh)
    for ctx in CTXS:
        for scale in [0.5, 0.02]:
            q, k, v = attention_inputs(rng, ctx, h, scale * np.sqrt(128))
            want = O.attention_decode(q, k, v, ctx, qh, kvh)
            atol = ATTENTION_ATOL_OF_VMAX * max_abs(v)
            what = f"attention {qh}/{kvh} ctx {ctx} scale {scale}"
            qb, kb, vb = bf16_bits(q), bf16_bits(k), bf16_bits(v)
            pages = (ctx + 15) // 16
            page_of = [int(p) for p in np.random.default_rng(ctx).permutation(pages + 2)[:pages]]
            per_head = bf16_vals(kernels.attention_decode(qb, kb, vb, ctx, h, page_of=page_of))
            assert_close(f"{what} per-head", per_head, want, atol, 0.0)
            for splits in [1, 4, 16, None]:
                split = kernels.attention_decode_split(qb, kb, vb, ctx, h, last_block=False, splits=splits,
                                                       page_of=page_of)
                assert_close(f"{what} split P {splits}", bf16_vals(split), want, atol, 0.0)
                if plan.grouped:
                    last = kernels.attention_decode_split(qb, kb, vb, ctx, h, last_block=True, splits=splits,
                                                          page_of=page_of)
                    assert (last == split).all(), f"{what} P {splits}: the two merges give the same bits"
                again = kernels.attention_decode_split(qb, kb, vb, ctx, h, last_block=False, splits=splits,
                                                       page_of=page_of)
                assert (again == split).all(), f"{what}: split-K is not deterministic"


@pytest.mark.parametrize("qh,kvh", [(1, 1), (2, 1), (16, 8), (32, 8), (64, 8)])
def test_fused_rope_attention_is_the_two_kernel_path_bit_for_bit(kernels, qh, kvh):
    """The engine's one-launch attention (QK-norm + RoPE + K/V write + split-K) gives the bits of
    the QK-norm/RoPE kernel followed by split-K on the same P and merge, writes the same K/V row
    into the page of position ctx - 1, and is the oracle's attention within tolerance."""
    from x0ne_core.ops import CacheAt, inv_freq
    h = H(qh, kvh)
    rng = O.Rng(470 + qh)
    theta, eps = 1e6, 1e-6
    for ctx in [1, 2, 16, 17, 64, 65, 255, 256, 257, 700, 2049]:
        qkv = rng.bf16s(h.q_dim + 2 * h.kv_dim, 3.0)
        qn, kn = rng.bf16s(128, 1.5), rng.bf16s(128, 1.5)
        k = rng.bf16s((ctx - 1) * h.kv_dim, 1.0)
        v = bf16s_with_edges(rng, (ctx - 1) * h.kv_dim, 4.0)
        pages = (ctx + 15) // 16
        page_of = [int(p) for p in np.random.default_rng(ctx).permutation(pages + 2)[:pages]]
        rope = kernels.qk_norm_rope_kv_write(bf16_bits(qkv), bf16_bits(qn), bf16_bits(kn), h, theta, eps,
                                             CacheAt(1, ctx, 0, ctx - 1))
        kb = np.concatenate([bf16_bits(k), rope.k_row])
        vb = np.concatenate([bf16_bits(v), rope.v_row])
        q_o, k_o, v_o = O.qk_norm_rope(qkv, qn, kn, inv_freq(128, theta), qh, kvh, 128, ctx - 1, eps)
        want = O.attention_decode(bf16_vals(rope.q), bf16_vals(kb), bf16_vals(vb), ctx, qh, kvh)
        atol = ATTENTION_ATOL_OF_VMAX * max(max_abs(v), max_abs(bf16_vals(rope.v_row)))
        what = f"fused {qh}/{kvh} ctx {ctx}"
        for splits in [1, 3, None]:
            for last_block in [True, False]:
                out, k_row, v_row = kernels.attention_rope_decode(
                    bf16_bits(qkv), bf16_bits(qn), bf16_bits(kn), eps, theta, bf16_bits(k), bf16_bits(v), ctx, h,
                    last_block=last_block, splits=splits, page_of=page_of)
                assert (k_row == rope.k_row).all() and (v_row == rope.v_row).all(), f"{what}: the K/V row"
                assert kernels.kv_rest_untouched, f"{what}: a K/V byte other than the new row changed"
                two = kernels.attention_decode_split(rope.q, kb, vb, ctx, h, last_block=last_block, splits=splits,
                                                     page_of=page_of)
                assert (out == two).all(), f"{what} P {splits} last_block {last_block}: not the two-kernel bits"
                assert_close(f"{what} P {splits}", bf16_vals(out), want, atol, 0.0)
        assert_close(f"{what} k row", bf16_vals(rope.k_row), k_o, ROPE_ATOL_OF_XMAX * max_abs(k_o) + BF16_ATOL,
                     BF16_RTOL)


@pytest.mark.parametrize("qh,kvh", [(1, 1), (2, 1), (4, 2), (16, 8), (32, 8), (64, 8)])
def test_batched_attention_is_each_sequence_alone_bit_for_bit(kernels, qh, kvh):
    """The batched step's attention (grid (kv_heads, P, B)): sequences at ragged positions, each
    in its own run of a shuffled page table over shared planes, get the bits the single-sequence
    fused kernel gives each alone on the same P, write the same K/V rows, and are the oracle's
    attention within tolerance."""
    from x0ne_core.ops import CacheAt
    h = H(qh, kvh)
    rng = O.Rng(490 + qh)
    theta, eps, max_ctx = 1e6, 1e-6, 1100
    ctxs = [1, 17, 256, 257, 1000]
    B = len(ctxs)
    qkv = [rng.bf16s(h.q_dim + 2 * h.kv_dim, 3.0) for _ in range(B)]
    qn, kn = rng.bf16s(128, 1.5), rng.bf16s(128, 1.5)
    ks = [rng.bf16s((c - 1) * h.kv_dim, 1.0) for c in ctxs]
    vs = [bf16s_with_edges(rng, (c - 1) * h.kv_dim, 4.0) for c in ctxs]
    for splits in [1, 4]:
        out, k_rows, v_rows = kernels.attention_rope_decode_batch(
            np.concatenate([bf16_bits(q) for q in qkv]), bf16_bits(qn), bf16_bits(kn), eps, theta,
            [bf16_bits(k) for k in ks], [bf16_bits(v) for v in vs], ctxs, h, splits, max_ctx, page_seed=5 + splits)
        assert kernels.kv_rest_untouched, f"batched {qh}/{kvh} P {splits}: a K/V byte other than the new rows changed"
        for b, ctx in enumerate(ctxs):
            what = f"batched {qh}/{kvh} P {splits} sequence {b} ctx {ctx}"
            one, k_row, v_row = kernels.attention_rope_decode(
                bf16_bits(qkv[b]), bf16_bits(qn), bf16_bits(kn), eps, theta, bf16_bits(ks[b]), bf16_bits(vs[b]), ctx,
                h, last_block=True, splits=splits)
            assert (out[b] == one).all(), f"{what}: not the single-sequence bits"
            assert (k_rows[b] == k_row).all() and (v_rows[b] == v_row).all(), f"{what}: the K/V row"
            rope = kernels.qk_norm_rope_kv_write(bf16_bits(qkv[b]), bf16_bits(qn), bf16_bits(kn), h, theta, eps,
                                                 CacheAt(1, ctx, 0, ctx - 1))
            assert (rope.k_row == k_row).all() and (rope.v_row == v_row).all(), f"{what}: the rope kernel's row"
            kb = np.concatenate([ks[b], bf16_vals(k_row)])
            vb = np.concatenate([vs[b], bf16_vals(v_row)])
            want = O.attention_decode(bf16_vals(rope.q), kb, vb, ctx, qh, kvh)
            assert_close(what, bf16_vals(out[b]), want, ATTENTION_ATOL_OF_VMAX * max_abs(vb), 0.0)


@pytest.mark.parametrize("ctx", [8192, 32768])
def test_config2_decode_attention_at_long_contexts(kernels, ctx):
    """BASELINE.json config 2 at its long contexts: 32 q / 8 kv heads, head_dim 128, bf16 Q, K and V
    drawn N(0, 1) from a seed, the keys in 16-position pages in a shuffled order, split-K at P 1,
    4, 16, the engine's plan, 64 and 128 (more slices than one merge chunk of 32): within
    max|V|/128 of the oracle (gpu_kernels.rs:437-599), the
    merge kernel and the last-block merge the same bits, a repeated launch the same bits; and
    the fused kernel (QK-norm, RoPE and the K/V write in front) on the same cache."""
    from x0ne_core.ops import CacheAt
    h = H(32, 8)
    g = np.random.default_rng(ctx)
    normal = lambda n: bf16_bits(g.standard_normal(n).astype(np.float32))
    q, k, v = normal(h.q_dim), normal(ctx * h.kv_dim), normal(ctx * h.kv_dim)
    pages = ctx // 16
    page_of = [int(p) for p in g.permutation(pages)]
    want = O.attention_decode(bf16_vals(q), bf16_vals(k), bf16_vals(v), ctx, 32, 8)
    atol = ATTENTION_ATOL_OF_VMAX * max_abs(bf16_vals(v))
    for splits in (1, 4, 16, None, 64, 128):
        outs = []
        for last_block in (True, False, True):
            out = kernels.attention_decode_split(q, k, v, ctx, h, last_block=last_block, splits=splits,
                                                 page_of=page_of)
            outs.append(out)
        what = f"config 2 ctx {ctx} P {splits}"
        assert_close(what, bf16_vals(outs[0]), want, atol, 0.0)
        assert (outs[0] == outs[1]).all(), f"{what}: the two merges differ"
        assert (outs[0] == outs[2]).all(), f"{what}: a repeat differs"
    qkv = np.concatenate([q, normal(2 * h.kv_dim)])
    qn, kn = bf16_bits(np.ones(128, np.float32)), bf16_bits(np.ones(128, np.float32))
    out, k_row, v_row = kernels.attention_rope_decode(qkv, qn, kn, 1e-6, 1e6, k[:(ctx - 1) * h.kv_dim],
                                                      v[:(ctx - 1) * h.kv_dim], ctx, h, page_of=page_of)
    assert kernels.kv_rest_untouched, f"fused ctx {ctx}: a K/V byte other than the new row changed"
    rope = kernels.qk_norm_rope_kv_write(qkv, qn, kn, h, 1e6, 1e-6, CacheAt(1, ctx, 0, ctx - 1))
    kb = np.concatenate([k[:(ctx - 1) * h.kv_dim], rope.k_row])
    vb = np.concatenate([v[:(ctx - 1) * h.kv_dim], rope.v_row])
    want = O.attention_decode(bf16_vals(rope.q), bf16_vals(kb), bf16_vals(vb), ctx, 32, 8)
    assert_close(f"config 2 fused ctx {ctx}", bf16_vals(out), want, ATTENTION_ATOL_OF_VMAX * max_abs(bf16_vals(vb)),
                 0.0)


@pytest.mark.parametrize("qh,kvh", [(1, 1), (2, 1), (16, 8), (32, 8), (64, 8)])
def test_exact_attention_is_the_f64_oracle_bit_for_bit(kernels, qh, kvh):
    """The exact mode's fused attention (f64 scores, softmax and sums) gives the bits of the f64
    oracle's attention rounded f64 -> f32 -> bf16, on the q and K/V row its own QK-norm/RoPE
    produced (which are the QK-norm/RoPE kernel's bits): at the engine's split plan and at split
    factors 1, 4 and 16 (f64 slice states merged by the last block in a fixed order), over pages
    in a shuffled order, up to 8192 keys."""
    from x0ne_core.ops import CacheAt
    h = H(qh, kvh)
    rng = O.Rng(490 + qh)
    theta, eps = 1e6, 1e-6
    total = differ = 0
    cases = [(ctx, None) for ctx in [1, 2, 17, 64, 65, 256, 257, 1000, 4097]]
    cases += [(ctx, p) for ctx in [300, 2049, 8192] for p in (1, 4, 16)]
    for ctx, splits in cases:
        qkv = rng.bf16s(h.q_dim + 2 * h.kv_dim, 3.0)
        qn, kn = rng.bf16s(128, 1.5), rng.bf16s(128, 1.5)
        k = rng.bf16s((ctx - 1) * h.kv_dim, 1.0)
        v = bf16s_with_edges(rng, (ctx - 1) * h.kv_dim, 4.0)
        v[~np.isfinite(v)] = 0.0
        pages = (ctx + 15) // 16
        page_of = [int(p) for p in np.random.default_rng(ctx).permutation(pages + 1)[:pages]]
        rope = kernels.qk_norm_rope_kv_write(bf16_bits(qkv), bf16_bits(qn), bf16_bits(kn), h, theta, eps,
                                             CacheAt(1, ctx, 0, ctx - 1))
        out, k_row, v_row = kernels.attention_rope_decode(bf16_bits(qkv), bf16_bits(qn), bf16_bits(kn), eps, theta,
                                                          bf16_bits(k), bf16_bits(v), ctx, h, page_of=page_of,
                                                          exact=True, splits=splits)
        assert (k_row == rope.k_row).all() and (v_row == rope.v_row).all(), f"ctx {ctx}: the K/V row"
        assert kernels.kv_rest_untouched, f"exact ctx {ctx}: a K/V byte other than the new row changed"
        kb = np.concatenate([bf16_bits(k), rope.k_row])
        vb = np.concatenate([bf16_bits(v), rope.v_row])
        want = bf16_bits(O.attention_decode(bf16_vals(rope.q), bf16_vals(kb), bf16_vals(vb), ctx, qh, kvh))
        total += want.size
        differ += int((out != want).sum())
    print(f"MEASURE exact attention {qh}/{kvh}: {differ} of {total} outputs differ from the f64 oracle's bits")
    assert differ == 0


@pytest.mark.parametrize("qh,kvh", [(1, 1), (2, 1), (16, 8), (32, 8), (64, 8)])
def test_exact_prefill_attention_is_the_f64_oracle_bit_for_bit(kernels, qh, kvh):
    """The exact mode's causal prefill (x0ne_attention_prefill_exact_g*_bf16: f64 scores,
    softmax and sums for every row of a pass) gives the bits of the f64 oracle's attention
    rounded f64 -> f32 -> bf16 for each row, whole and from a chunk boundary, over pages in a
    shuffled order, across block boundaries of rows and tiles of keys."""
    h = H(qh, kvh)
    rng = O.Rng(520 + qh)
    total = differ = 0
    for t, pos0 in [(1, 0), (2, 0), (17, 0), (64, 0), (65, 0), (130, 0), (130, 1), (130, 64), (513, 0),
                    (513, 448), (1025, 1000), (4097, 3990)]:
        q = rng.bf16s((t - pos0) * h.q_dim, 3.0)
        k = rng.bf16s(t * h.kv_dim, 3.0)
        v = bf16s_with_edges(rng, t * h.kv_dim, 4.0)
        v[~np.isfinite(v)] = 0.0
        m = t - pos0
        rows = list(range(m)) if m <= 130 else sorted(set([0, 1, m - 1, m // 2] + [rng.below(m) for _ in range(6)]))
        pages = (t + 15) // 16
        page_of = [int(p) for p in np.random.default_rng(t).permutation(pages + 2)[:pages]]
        got = kernels.attention_prefill_at(bf16_bits(q), bf16_bits(k), bf16_bits(v), t, pos0, h, rows,
                                           page_of=page_of, exact=True)
        want = O.attention_rows(q, k, v, pos0, qh, kvh, 128, rows)
        for r, g, w in zip(rows, got, want):
            wb = bf16_bits(w)
            total += wb.size
            bad = int((g != wb).sum())
            differ += bad
            assert bad == 0, f"exact prefill {qh}/{kvh} t {t} pos0 {pos0} row {r}: {bad} outputs differ"
    print(f"MEASURE exact prefill attention {qh}/{kvh}: {differ} of {total} outputs differ from the f64 oracle's bits")


def test_decode_attention_on_one_key_a_dominant_key_and_equal_keys(kernels):
    h = H(4, 2)
    rng = O.Rng(450)
    q = rng.bf16s(h.q_dim, 4.0)
    v = rng.bf16s(300 * h.kv_dim, 4.0)
    kk = rng.bf16s(300 * h.kv_dim, 4.0)
    for split in [False, True]:
        def run(kk_, v_, ctx):
            f = kernels.attention_decode_split if split else kernels.attention_decode
            return bf16_vals(f(bf16_bits(q), bf16_bits(kk_), bf16_bits(v_), ctx, h))
        one = run(kk, v, 1)
        for head in range(4):
            kh = head // 2
            assert (bf16_bits(one[head * 128:(head + 1) * 128]) == bf16_bits(v[kh * 128:(kh + 1) * 128])).all()
        dom = kk.copy()
        for kh in range(2):
            dom[137 * h.kv_dim + kh * 128:137 * h.kv_dim + (kh + 1) * 128] = O.bf16_round(
                q[kh * 256:kh * 256 + 128] * 16.0)
        assert_close(f"dominant key split {split}", run(dom, v, 300), O.attention_decode(q, dom, v, 300, 4, 2),
                     ATTENTION_ATOL_OF_VMAX * 4.0, 0.0)
        same = np.tile(kk[:h.kv_dim], 300)
        assert_close(f"equal keys split {split}", run(same, v, 300), O.attention_decode(q, same, v, 300, 4, 2),
                     ATTENTION_ATOL_OF_VMAX * 4.0, 0.0)
    from x0ne_core import FormatError
    with pytest.raises(FormatError):
        kernels.attention_decode(bf16_bits(q), bf16_bits(kk), bf16_bits(v), 0, h)
    with pytest.raises(FormatError):
        kernels.attention_decode(bf16_bits(q), bf16_bits(kk), bf16_bits(v), 301, h)


@pytest.mark.parametrize("qh,kvh", [(2, 1), (4, 2), (16, 8), (32, 8), (8, 8), (16, 2)])
def test_prefill_attention_is_the_oracle_whole_and_from_a_chunk_boundary(kernels, qh, kvh):
    """Both prefill kernels (per q head and row on the vector units; the matrix-core kernel per
    group of rows and heads), whole and from a chunk boundary, against the oracle's causal rows."""
    h = H(qh, kvh)
    rng = O.Rng(500 + qh)
    for t in [1, 2, 15, 16, 17, 63, 64, 65, 511, 513, 1025]:
        q = rng.bf16s(t * h.q_dim, 0.3 * np.sqrt(128))
        k = rng.bf16s(t * h.kv_dim, 0.3 * np.sqrt(128))
        v = bf16s_with_edges(rng, t * h.kv_dim, 4.0)
        atol = ATTENTION_ATOL_OF_VMAX * max_abs(v)
        rows = sorted(set([0, t - 1, t // 2, rng.below(t)]))
        want = O.attention_rows(q, k, v, 0, qh, kvh, 128, rows)
        for grouped in [False, True]:
            got = kernels.attention_prefill_rows(bf16_bits(q), bf16_bits(k), bf16_bits(v), t, h, rows, grouped=grouped)
            for r, g, w in zip(rows, got, want):
                assert_close(f"prefill {qh}/{kvh} t {t} row {r} grouped {grouped}", bf16_vals(g), w, atol, 0.0)
        # The panel-output variant: the grouped kernel's bits at the panel positions.
        every = list(range(t))
        rowwise = kernels.attention_prefill_rows(bf16_bits(q), bf16_bits(k), bf16_bits(v), t, h, every, grouped=True)
        panel = kernels.attention_prefill_rows(bf16_bits(q), bf16_bits(k), bf16_bits(v), t, h, every, panel=True)
        assert (np.array(panel) == np.array(rowwise)).all(), f"prefill panel {qh}/{kvh} t {t}"
        for pos0 in sorted(set([0, 1, t // 2, t - 1])):
            if pos0 >= t:
                continue
            tail = list(range(0, t - pos0, max(1, (t - pos0) // 5)))
            want = O.attention_rows(q[pos0 * h.q_dim:], k, v, pos0, qh, kvh, 128, tail)
            for grouped in [False, True]:
                got = kernels.attention_prefill_at(bf16_bits(q[pos0 * h.q_dim:]), bf16_bits(k), bf16_bits(v), t,
                                                   pos0, h, tail, grouped=grouped)
                for r, g, w in zip(tail, got, want):
                    assert_close(f"prefill at {pos0} t {t} row {r} grouped {grouped}", bf16_vals(g), w, atol, 0.0)


def test_the_isolated_attention_timing_rotates_distinct_planes(kernels):
    """BASELINE.json config 2's harness (x0ne_gpu_time_attention): it runs the grouped split-K
    kernel over more than 512 MiB of distinct K/V planes and reports a positive kernel time."""
    for ctx, p in [(64, 1), (1024, 4)]:
        us, planes = kernels.gpu.time_attention(32, 8, ctx, p, 4, 0)
        plane = (ctx + 15) // 16 * 8 * 16 * 128 * 2
        assert us > 0 and planes >= 2 and 2 * plane * planes > 512 << 20, (ctx, p, us, planes)


@pytest.mark.parametrize("seed", range(20))
def test_swiglu_is_the_oracle(kernels, seed):
    rng = O.Rng(600 + seed)
    inter = rng.pick([1, 2, 7, 8, 255, 256, 3072, 12288])
    scale = rng.pick([1.0, 8.0, 40.0, 200.0])
    gu = bf16s_with_edges(rng, 2 * inter, scale)
    got = bf16_vals(kernels.swiglu(bf16_bits(gu)))
    assert_close(f"swiglu seed {seed} inter {inter}", got, O.swiglu(gu), BF16_ATOL, BF16_RTOL)
    rows = rng.pick([1, 2, 5])
    many = rng.bf16s(rows * 2 * min(inter, 256), 8.0)
    got = bf16_vals(kernels.swiglu_rows(bf16_bits(many), rows))
    want = np.concatenate([O.swiglu(r) for r in many.reshape(rows, -1)])
    assert_close(f"swiglu rows seed {seed}", got, want, BF16_ATOL, BF16_RTOL)
    # The panel-output variant (inter a multiple of 8): the same bits at the panel positions.
    if inter % 8 == 0:
        prow = rng.pick([1, 15, 17, 40])
        gu2 = bf16s_with_edges(rng, prow * 2 * inter, scale)
        rowwise = kernels.swiglu_rows(bf16_bits(gu2), prow)
        assert (kernels.swiglu_rows(bf16_bits(gu2), prow, panel=True) == rowwise).all(), f"swiglu panel seed {seed}"


def test_swiglu_special_values(kernels):
    s = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 200.0, -200.0, bf16_vals(1)[0], bf16_vals(0x7F7F)[0],
                  bf16_vals(0xFF7F)[0]], np.float32)
    s16 = np.concatenate([s, s[:6]])  # 16 values: the 16-byte path (inter a multiple of 8)
    for gate, up in [(s, np.full(s.size, 2.0, np.float32)), (np.ones(s.size, np.float32), s),
                     (s16, np.full(16, 2.0, np.float32)), (np.ones(16, np.float32), s16)]:
        gu = np.concatenate([gate, up])
        got = bf16_vals(kernels.swiglu(bf16_bits(gu)))
        want = O.bf16_round(O.swiglu(gu))
        assert (np.isnan(got) == np.isnan(want)).all()
        fin = ~np.isnan(want)
        assert ((got[fin] == want[fin]) | (np.abs(got[fin] - want[fin]) <= BF16_RTOL * np.abs(want[fin]) + 1e-30)).all()


def test_argmax_is_the_first_largest_and_a_nan_row_has_none(kernels):
    from x0ne_core import FormatError, GpuError
    rng = O.Rng(700)
    for rnd in range(100):
        n = rng.pick([1, 2, 3, 63, 64, 65, 1023, 1024, 1025, 2047, 4096, 151936])
        if rng.chance(2):
            row = np.array([rng.below(4) - 2.0 for _ in range(min(n, 4096))] + [0.0] * max(0, n - 4096), np.float32)
        else:
            row = rng.f32s(n, 50.0)
        for _ in range(rng.below(4)):
            row[rng.below(n)] = rng.pick([0.0, -0.0, np.inf, -np.inf, np.finfo(np.float32).max,
                                          np.finfo(np.float32).min])
        assert kernels.argmax(row) == O.argmax(row), f"round {rnd}: {n} values"
        for at in [0, n - 1]:
            moved = row.copy()
            moved[at] = np.inf
            assert kernels.argmax(moved) == O.argmax(moved)
        nan = row.copy()
        nan[rng.below(n)] = np.nan
        with pytest.raises(GpuError):
            kernels.argmax(nan)
    assert kernels.argmax(np.full(5, -np.inf, np.float32)) == 0
    assert kernels.argmax(np.array([-0.0, 0.0], np.float32)) == 0
    with pytest.raises(FormatError):
        kernels.argmax(np.zeros(0, np.float32))


def test_sliced_argmax_picks_what_the_one_block_argmax_picks(kernels):
    """The batched step's argmax (rows cut in slices, then a pick over the slices) against the
    oracle's first largest, with ties straddling slice boundaries, infinities, a NaN row, a row
    of -inf, and slices past the row's end; every position advances by one."""
    rng = O.Rng(710)
    for n, slices in [(151936, 64), (1000, 64), (65, 64), (7, 64), (4096, 3), (1, 1)]:
        rows = []
        for r in range(6):
            row = rng.f32s(n, 30.0) if r % 2 else np.array([rng.below(3) - 1.0 for _ in range(n)], np.float32)
            rows.append(row)
        per = -(-n // slices)
        if n > 2 * per:
            rows[2][[per - 1, per]] = np.float32(1e30)  # a tie across a slice boundary: the first wins
        rows[3][n - 1] = np.inf
        rows[4][:] = -np.inf
        nan_row = rng.f32s(n, 1.0)
        nan_row[rng.below(n)] = np.nan
        rows.append(nan_row)
        logits = np.stack(rows)
        pos = np.arange(len(rows), dtype=np.uint32) * 1000 + 5
        toks, after = kernels.argmax_rows_sliced(logits, slices, pos)
        for r in range(len(rows) - 1):
            assert toks[r] == O.argmax(logits[r]), f"n {n} slices {slices} row {r}"
        assert toks[-1] == 0xFFFFFFFF, "a NaN row has no pick"
        assert (after == pos + 1).all()


def test_advance_adds_one(kernels):
    for v in [0, 1, 511, 512, 131071, 2**32 - 2]:
        assert kernels.advance(v) == v + 1


@pytest.mark.parametrize("seed", range(40))
def test_moe_kernels_are_the_reference(kernels, seed):
    """gpu_kernels.rs:841-914: the routing (ids exact, weights within 1e-6 + 1e-5 relative) over
    1 to 1024 experts with ties and a non-finite logit now and then; the expert GEMVs through
    the routed ids (an undefined row included) in f32 and bf16; the weighted combination."""
    rng = O.Rng(800 + seed)
    experts = rng.pick([1, 2, 8, 128, 1024])
    top_k = rng.range(1, min(experts, 32))
    rows = rng.range(1, 9)
    if rng.chance(3):
        logits = np.array([float(rng.below(3)) for _ in range(rows * experts)], np.float32)
    else:
        logits = np.asarray(rng.f32s(rows * experts, 6.0), np.float32)
    if rng.chance(3):
        logits[rng.below(rows * experts)] = rng.pick([np.nan, np.inf, -np.inf])
    ids, w = kernels.moe_route(logits, experts, top_k)
    want_ids, want_w = O.moe_route(logits, experts, top_k)
    what = f"seed {seed}: {experts} experts, top {top_k}, {rows} rows"
    assert (ids == want_ids).all(), what
    assert_close(f"moe weights {what}", w, want_w, 1e-6, 1e-5)
    r, cols = rng.pick([1, 8, 24]), 8 * rng.range(1, 8)
    small = min(experts, 8)
    ids = np.array([i if i == O.MOE_NO_EXPERT or i < small else i % small for i in ids.tolist()], np.uint32)
    wt = np.asarray(rng.bf16s(small * r * cols, 1.0), np.float32)
    x = np.asarray(rng.bf16s(rows * cols, 2.0), np.float32)
    want = O.moe_gemv(wt, small, r, cols, ids, x, top_k)
    for f32_out in (True, False):
        got = kernels.moe_gemv(bf16_bits(wt), small, r, cols, ids, bf16_bits(x), top_k, f32_out)
        assert_close(f"moe gemv {what} f32 {f32_out}", got, want, 1e-4, 1e-4 if f32_out else BF16_RTOL)
    hidden = 8 * rng.range(1, 16)
    y = np.asarray(rng.f32s(rows * top_k * hidden, 3.0), np.float32)
    wts = np.asarray(rng.f32s(rows * top_k, 1.0), np.float32)
    got = bf16_vals(kernels.moe_combine(y, wts, hidden, top_k))
    assert_close(f"moe combine {what}", got, O.moe_combine(y, wts, hidden, top_k), 1e-4, BF16_RTOL)


@pytest.mark.parametrize("seed", range(8))
def test_the_fused_moe_projections_are_the_composed_oracle(kernels, seed):
    """The kernels the MoE step runs: [gate; up] with SwiGLU behind against the oracle's expert
    GEMV then swiglu (oracle/src/lib.rs:284-312, :205-214), and down with the weighted
    combination behind against the oracle's f32 expert GEMV then combination (:314-329); the
    projections within the GEMV tolerance, each activation within the SwiGLU of its gate and up
    intervals, the combination within one bf16 rounding past them; a slot without an expert gives
    NaN."""
    rng = O.Rng(850 + seed)
    experts = rng.pick([2, 8, 64])
    top_k = rng.range(1, min(experts, 8))
    inter = 8 * rng.range(1, 40)
    hidden = 8 * rng.range(1, 64)
    wgu = np.asarray(rng.bf16s(experts * 2 * inter * hidden, 0.2), np.float32)
    wd = np.asarray(rng.bf16s(experts * hidden * inter, 0.2), np.float32)
    x = np.asarray(rng.bf16s(hidden, 2.0), np.float32)
    ids = np.array([rng.below(experts) for _ in range(top_k)], np.uint32)
    if seed == 3:
        ids[-1] = O.MOE_NO_EXPERT
    wts = np.asarray(rng.f32s(top_k, 1.0), np.float32)
    what = f"seed {seed}: {experts} experts, top {top_k}, inter {inter}, hidden {hidden}"
    gu = O.moe_gemv(wgu, experts, 2 * inter, hidden, ids, x, top_k).reshape(top_k, 2 * inter)
    act = bf16_vals(kernels.moe_gate_up_swiglu(bf16_bits(wgu), experts, inter, hidden, ids, bf16_bits(x)))
    act = act.reshape(top_k, inter)
    want_act = O.bf16_round(np.stack([O.swiglu(O.bf16_round(gu[s])) for s in range(top_k)]))
    for s in range(top_k):
        if ids[s] == O.MOE_NO_EXPERT:
            assert np.isnan(act[s]).all(), f"{what}: slot {s} without an expert"
            continue
        e = int(ids[s])
        mag = O.gemv_magnitude(wgu[e * 2 * inter * hidden:(e + 1) * 2 * inter * hidden], 2 * inter, hidden, x)
        tol = F32_RTOL * mag + 1e-30
        for i in range(inter):
            g, u = float(gu[s, i]), float(gu[s, inter + i])
            cands = [O.swiglu(np.array([gg, uu], np.float32))[0]
                     for gg in O.bf16_round(np.array([g - tol[i], g + tol[i]], np.float32))
                     for uu in O.bf16_round(np.array([u - tol[inter + i], u + tol[inter + i]], np.float32))]
            lo, hi = O.bf16_round(np.float32(min(cands)))[0], O.bf16_round(np.float32(max(cands)))[0]
            assert lo - abs(lo) * 2 ** -7 <= act[s, i] <= hi + abs(hi) * 2 ** -7, f"{what}: act [{s}][{i}]"
    exact = float((bf16_bits(act) == bf16_bits(want_act)).mean())
    ok = ids != O.MOE_NO_EXPERT
    y = O.moe_gemv(wd, experts, hidden, inter, ids, want_act, 1).reshape(top_k, hidden)
    out = bf16_vals(kernels.moe_down_combine(bf16_bits(wd), experts, hidden, inter, ids, wts,
                                             bf16_bits(want_act.ravel())))
    want = O.moe_combine(y, wts, hidden, top_k)
    if not ok.all():
        assert np.isnan(out).all(), f"{what}: a slot without an expert makes the row NaN"
    else:
        mags = np.stack([O.gemv_magnitude(wd[int(e) * hidden * inter:(int(e) + 1) * hidden * inter], hidden, inter,
                                          want_act[s]) for s, e in enumerate(ids)])
        atol = F32_RTOL * (np.abs(wts)[:, None] * mags).sum(0) + 1e-6
        r = np.abs(out.astype(np.float64) - want) / (atol + BF16_RTOL * np.abs(want))
        print(f"MEASURE moe down + combination {what}: worst ratio {r.max():.4f}")
        assert (r <= 1.0).all(), f"{what}: output {int(np.argmax(r))}"
    print(f"MEASURE fused moe {what}: {exact:.4f} of the activations bit-equal to the oracle's")


@pytest.mark.parametrize("seed", range(8))
def test_the_exact_moe_projections_are_the_oracle_bit_for_bit(kernels, seed):
    """The exact mode's MoE kernels against the oracle's composition, bit for bit: [gate; up]
    with SwiGLU behind, each sum in f64 rounded to f32, is the oracle's expert GEMV then
    bf16 and swiglu (oracle/src/lib.rs:284-312, :205-214); down with the f64 combination behind
    is the oracle's f32 expert GEMV then combination (:314-329) rounded to bf16. Rows of up to
    1592 columns, so the lanes' two-chunk loop runs; a slot without an expert gives NaN."""
    g = np.random.default_rng(870 + seed)
    experts = int(g.choice([2, 8]))
    top_k = int(g.integers(1, experts + 1))
    inter, hidden = 8 * int(g.integers(1, 100)), 8 * int(g.integers(1, 200))
    if seed == 0:
        inter, hidden = 8, 8
    bf = lambda n, sd: O.bf16_round(g.normal(0, sd, n).astype(np.float32))
    wgu, wd = bf(experts * 2 * inter * hidden, 0.2), bf(experts * hidden * inter, 0.2)
    x = bf(hidden, 2.0)
    if seed == 1:
        x[:] = 0.0
        x[::3] = -0.0
    ids = g.integers(0, experts, top_k).astype(np.uint32)
    if seed == 3:
        ids[-1] = O.MOE_NO_EXPERT
    wts = g.uniform(0.0, 1.0, top_k).astype(np.float32)
    what = f"seed {seed}: {experts} experts, top {top_k}, inter {inter}, hidden {hidden}"
    gu = O.moe_gemv(wgu, experts, 2 * inter, hidden, ids, x, top_k).reshape(top_k, 2 * inter)
    act = kernels.moe_gate_up_swiglu(bf16_bits(wgu), experts, inter, hidden, ids, bf16_bits(x), exact=True)
    act = act.reshape(top_k, inter)
    want_act = np.stack([O.bf16_round(O.swiglu(O.bf16_round(gu[s]))) for s in range(top_k)])
    for s in range(top_k):
        if ids[s] == O.MOE_NO_EXPERT:
            assert np.isnan(bf16_vals(act[s])).all(), f"{what}: slot {s} without an expert"
            continue
        assert (act[s] == bf16_bits(want_act[s])).all(), f"{what}: slot {s} activations"
    act_in = np.where(np.isnan(want_act), np.float32(0.5), want_act).astype(np.float32)
    y = O.moe_gemv(wd, experts, hidden, inter, ids, act_in, 1).reshape(top_k, hidden)
    out = kernels.moe_down_combine(bf16_bits(wd), experts, hidden, inter, ids, wts, bf16_bits(act_in.ravel()),
                                   exact=True)
    if (ids == O.MOE_NO_EXPERT).any():
        assert np.isnan(bf16_vals(out)).all(), f"{what}: a slot without an expert makes the row NaN"
    else:
        want = bf16_bits(O.bf16_round(O.moe_combine(y, wts, hidden, top_k)))
        assert (out == want).all(), f"{what}: output {int(np.argmax(out != want))}"


def test_moe_routing_refuses_what_the_kernel_does_not_take(kernels):
    """gpu_kernels.rs:915-930."""
    from x0ne_core import FormatError
    for experts, top_k, n in [(0, 1, 8), (1025, 1, 1025), (8, 0, 8), (8, 9, 8), (64, 33, 64), (8, 2, 7), (8, 2, 0)]:
        with pytest.raises(FormatError):
            kernels.moe_route(np.zeros(n, np.float32), experts, top_k)
