"""The fused decode GEMV instances, each driven alone (x0ne_gpu_gemv_fused), against the composed
oracle: add_rmsnorm -> gemv -> (swiglu | argmax), oracle/src/lib.rs:50-70, :123-134, :205-230.

These are the kernels the decode step runs for its projections; the reference runs the same
work as separate kernels around cuBLAS, checked at gpu_kernels.rs:97-191 (add_rmsnorm: residual
bit for bit, output within 1/128), :331-393 (GEMV: within 1e-5 of the sum of |w x| plus the bf16
rounding), :698-774 (SwiGLU within 1/128) and :778-839 (argmax bit for bit, ties to the lowest
index, a NaN row gives 0xFFFFFFFF; advance). The f32-sum instances are held to those tolerances;
the f64-sum instances (the exact mode) add each exact product in f64 as the oracle does, so
their outputs are the oracle's bits. Widths: the hidden sizes of Qwen3-0.6B/8B/32B for the norm
prologues (1024, 4096, 5120), and also their attention and MLP widths (12288, 25600) where x is
given; and two rows narrower than the 0.6B's, which take the same narrow tiles (two chunks per
lane): 8 (one chunk in all) and 520 (65 chunks, the 65th in lane 0's second slot)."""
import numpy as np
import pytest

from common import BF16_RTOL, F32_RTOL, O, bf16_bits, bf16_vals, bf16s_with_edges

pytestmark = pytest.mark.gpu

NORM_WIDTHS = [8, 520, 1024, 4096, 5120]
X_WIDTHS = [8, 520, 1024, 4096, 5120, 12288, 25600]
NO_TOKEN = 0xFFFFFFFF


@pytest.fixture(scope="module")
def K():
    from x0ne_core.ops import Kernels
    return Kernels()


def normed(residual, delta, norm_w, eps):
    """The oracle's add + RMSNorm: (new f32 residual, x rounded to bf16)."""
    r, out = O.add_rmsnorm(residual, delta, norm_w, eps)
    return r, O.bf16_round(out)


def gemv_bound(mag, want, rounded):
    """gpu_kernels.rs:331-393: 1e-5 of sum |w x|, plus one bf16 rounding when the output is bf16."""
    return F32_RTOL * mag + ((BF16_RTOL * np.abs(want).astype(np.float64) + 1e-6) if rounded else 1e-30)


def check_gemv(what, got, want, mag, rounded, f64):
    got = np.asarray(got, np.float64)
    want64 = np.asarray(want, np.float64)
    if f64:
        differ = int((np.asarray(got, np.float32).view(np.uint32) != np.asarray(want, np.float32).view(np.uint32)).sum())
        print(f"MEASURE {what}: {differ} of {got.size} outputs differ from the oracle's bits")
        assert differ == 0, what
        return
    r = np.abs(got - want64) / gemv_bound(mag, want64, rounded)
    print(f"MEASURE {what}: worst ratio {r.max():.4f}")
    assert (r <= 1.0).all(), f"{what}: row {int(np.argmax(r))} got {got[np.argmax(r)]} want {want64[np.argmax(r)]}"


def data(seed, rows, cols, scale=1.0):
    rng = O.Rng(seed)
    w = bf16s_with_edges(rng, rows * cols, 0.05 * scale)
    residual = (rng.f32s(cols, 2.0)).astype(np.float32)
    delta = rng.bf16s(cols, 1.0)
    norm_w = O.bf16_round(np.float32(1.0) + rng.f32s(cols, 0.25))
    return w, residual, delta, norm_w


@pytest.mark.parametrize("f64", [False, True], ids=["f32", "f64"])
@pytest.mark.parametrize("cols", NORM_WIDTHS)
def test_the_normed_projection_is_add_rmsnorm_then_gemv(K, cols, f64):
    """QKV's instance (prologue add + RMSNorm, bf16 out) and its f32-out twin: the new residual is
    the oracle's f32 add bit for bit, the output the oracle's GEMV of the normed row."""
    eps = 1e-6
    for rows in (7, 1031, 3 * cols // 2):
        w, residual, delta, norm_w = data(1000 + rows + cols, rows, cols)
        r_want, x = normed(residual, delta, norm_w, eps)
        want = O.gemv(w, rows, cols, x)
        mag = O.gemv_magnitude(w, rows, cols, x)
        for epi, rounded in ((K.EPI_BF16, True), (K.EPI_F32, False)):
            out = K.gemv_fused(bf16_bits(w), rows, cols, K.PRO_NORM, epi, f64, residual=residual,
                               delta=bf16_bits(delta), norm_w=bf16_bits(norm_w), eps=eps)
            what = f"norm+gemv {rows}x{cols} {'bf16' if rounded else 'f32'} out, {'f64' if f64 else 'f32'} sums"
            assert (out["residual"].view(np.uint32) == r_want.view(np.uint32)).all(), f"{what}: residual"
            got = bf16_vals(out["y"]) if rounded else out["y"]
            check_gemv(what, got, O.bf16_round(want) if (rounded and f64) else want, mag, rounded, f64)


@pytest.mark.parametrize("f64", [False, True], ids=["f32", "f64"])
@pytest.mark.parametrize("cols", NORM_WIDTHS)
def test_the_first_layers_projection_is_embedding_then_norm_then_gemv(K, cols, f64):
    """Layer 0's QKV instance: the embedding row of the token (a token past the table gives a zero
    row, embedding.cu:5-17) on a zero residual, normed, projected; the residual out is the row."""
    eps = 1e-6
    vocab, rows = 97, 523
    rng = O.Rng(2000 + cols)
    table = rng.bf16s(vocab * cols, 1.0)
    w = bf16s_with_edges(rng, rows * cols, 0.05)
    norm_w = O.bf16_round(np.float32(1.0) + rng.f32s(cols, 0.25))
    for token in (0, 5, vocab - 1, vocab, 2 ** 32 - 1):
        row = O.embedding(table, cols, token)
        r_want, x = normed(np.zeros(cols, np.float32), row, norm_w, eps)
        want = O.gemv(w, rows, cols, x)
        mag = O.gemv_magnitude(w, rows, cols, x)
        out = K.gemv_fused(bf16_bits(w), rows, cols, K.PRO_EMBED_NORM, K.EPI_BF16, f64, embed=bf16_bits(table),
                           token=token, vocab=vocab, norm_w=bf16_bits(norm_w), eps=eps)
        what = f"embed+norm+gemv token {token} {rows}x{cols}, {'f64' if f64 else 'f32'} sums"
        assert (out["residual"].view(np.uint32) == r_want.view(np.uint32)).all(), f"{what}: residual"
        if token >= vocab:
            # zero values; a row of weights that are all negative sums its -0.0 products to -0.0
            assert (out["residual"] == 0).all() and (bf16_vals(out["y"]) == 0).all(), what
        check_gemv(what, bf16_vals(out["y"]), O.bf16_round(want) if f64 else want, mag, True, f64)


def swiglu_interval(g_lo, g_hi, u_lo, u_hi):
    """Smallest and largest of bf16(silu(g) u) over bf16 g in [g_lo, g_hi] and u in [u_lo, u_hi]
    (silu(g) u is monotone in u, and in g except around silu's minimum at g = -1.2785)."""
    cand = []
    for g in (g_lo, g_hi, np.clip(-1.2784645, g_lo, g_hi)):
        for u in (u_lo, u_hi):
            cand.append(O.swiglu(np.array([g, u], np.float32))[0])
    cand = np.array(cand, np.float64)
    return O.bf16_round(np.float32(cand.min()))[0], O.bf16_round(np.float32(cand.max()))[0]


@pytest.mark.parametrize("f64", [False, True], ids=["f32", "f64"])
@pytest.mark.parametrize("cols", NORM_WIDTHS)
def test_the_gate_up_projection_is_norm_then_gemv_then_swiglu(K, cols, f64):
    """The dominant kernel's instance: add + RMSNorm, [gate; up] GEMV, act = bf16(silu(bf16 g)
    bf16 u). The f64 instance gives the oracle's bits; the f32 one lies within the activations
    its gate and up may take within the GEMV tolerance (the swiglu of every bf16 value in each
    interval), so a wrong pairing of gate and up rows fails it."""
    eps = 1e-6
    inter = 1500 if cols != 4096 else 3072
    rows = 2 * inter
    w, residual, delta, norm_w = data(3000 + cols, rows, cols)
    r_want, x = normed(residual, delta, norm_w, eps)
    gu = O.gemv(w, rows, cols, x)
    mag = O.gemv_magnitude(w, rows, cols, x)
    out = K.gemv_fused(bf16_bits(w), rows, cols, K.PRO_NORM, K.EPI_SWIGLU, f64, residual=residual,
                       delta=bf16_bits(delta), norm_w=bf16_bits(norm_w), eps=eps)
    what = f"norm+gate_up+swiglu inter {inter} cols {cols}, {'f64' if f64 else 'f32'} sums"
    assert (out["residual"].view(np.uint32) == r_want.view(np.uint32)).all(), f"{what}: residual"
    got = bf16_vals(out["y"])
    want = O.bf16_round(O.swiglu(O.bf16_round(gu)))
    if f64:
        differ = int((bf16_bits(got) != bf16_bits(want)).sum())
        print(f"MEASURE {what}: {differ} of {inter} activations differ from the oracle's bits")
        assert differ == 0
        return
    tol = F32_RTOL * mag
    bad = 0
    for i in range(inter):
        g, u = float(gu[i]), float(gu[inter + i])
        lo, hi = swiglu_interval(O.bf16_round(np.float32(g - tol[i]))[0], O.bf16_round(np.float32(g + tol[i]))[0],
                                 O.bf16_round(np.float32(u - tol[inter + i]))[0],
                                 O.bf16_round(np.float32(u + tol[inter + i]))[0])
        if not (min(lo, hi) <= got[i] <= max(lo, hi)):
            bad += 1
            print(f"activation {i}: got {got[i]} outside [{lo}, {hi}] (g {g}, u {u})")
    exact = int((bf16_bits(got) == bf16_bits(want)).sum())
    print(f"MEASURE {what}: {exact} of {inter} activations equal to the oracle's bits, {bad} outside the interval")
    assert bad == 0


@pytest.mark.parametrize("f64", [False, True], ids=["f32", "f64"])
@pytest.mark.parametrize("cols", NORM_WIDTHS)
def test_the_lm_head_is_norm_then_gemv_then_argmax_and_advance(K, cols, f64):
    """The LM head's instance: final norm, f32 logits, the first largest index into the token and
    pos + 1 (advance) or pos (no advance), the block counter left at 0; logits within the GEMV
    tolerance (f32 sums) or the oracle's bits (f64 sums); the token the first maximum of the
    device's own logits, and the oracle's when its margin exceeds twice the tolerance."""
    eps = 1e-6
    vocab = 20011
    w, residual, delta, norm_w = data(4000 + cols, vocab, cols, scale=4.0)
    r_want, x = normed(residual, delta, norm_w, eps)
    want = O.gemv(w, vocab, cols, x)
    mag = O.gemv_magnitude(w, vocab, cols, x)
    for advance, pos in ((True, 41), (False, 7)):
        out = K.gemv_fused(bf16_bits(w), vocab, cols, K.PRO_NORM, K.EPI_ARGMAX, f64, residual=residual,
                           delta=bf16_bits(delta), norm_w=bf16_bits(norm_w), eps=eps, advance=advance, pos=pos)
        what = f"norm+lm_head+argmax {vocab}x{cols}, {'f64' if f64 else 'f32'} sums, advance {advance}"
        assert (out["residual"].view(np.uint32) == r_want.view(np.uint32)).all(), f"{what}: residual"
        check_gemv(what, out["y"], want, mag, False, f64)
        assert out["token"] == O.argmax(out["y"]), f"{what}: the first maximum of its own logits"
        order = np.argsort(-want.astype(np.float64), kind="stable")
        tol = F32_RTOL * float(mag.max())
        if float(want[order[0]]) - float(want[order[1]]) > 2 * tol:
            assert out["token"] == int(order[0]), what
        assert out["pos"] == pos + (1 if advance else 0), what
        assert out["counter"] == 0, f"{what}: counter left at {out['counter']}"
        print(f"MEASURE {what}: token {out['token']} over {out['blocks']} blocks")


@pytest.mark.parametrize("f64", [False, True], ids=["f32", "f64"])
def test_the_lm_head_argmax_ties_nans_and_single_blocks(K, f64):
    """argmax.cu:11-58 through the fused head: equal maxima in different blocks go to the lowest
    index; a NaN anywhere in the row gives 0xFFFFFFFF; a row of -inf logits picks index 0."""
    eps = 1e-6
    cols, vocab = 1024, 9000
    rng = O.Rng(4500)
    residual = rng.f32s(cols, 1.0).astype(np.float32)
    delta = rng.bf16s(cols, 1.0)
    norm_w = np.ones(cols, np.float32)
    r_want, x = normed(residual, delta, norm_w, eps)
    base = rng.bf16s(cols, 0.01)
    w = np.tile(O.bf16_round(base), vocab).astype(np.float32)  # every logit equal
    out = K.gemv_fused(bf16_bits(w), vocab, cols, K.PRO_NORM, K.EPI_ARGMAX, f64, residual=residual,
                       delta=bf16_bits(delta), norm_w=bf16_bits(norm_w), eps=eps, advance=True, pos=0)
    assert out["token"] == 0 and out["pos"] == 1, "all equal: index 0"
    s0 = float(O.gemv(O.bf16_round(base), 1, cols, x)[0])
    assert s0 != 0.0
    big = O.bf16_round(base * np.float32(2.0 if s0 > 0 else -2.0))  # a larger logit
    for rows_at in ([8999], [17, 8999], [4500, 6000, 8999]):
        w2 = w.reshape(vocab, cols).copy()
        for r in rows_at:
            w2[r] = big
        out = K.gemv_fused(bf16_bits(w2.ravel()), vocab, cols, K.PRO_NORM, K.EPI_ARGMAX, f64, residual=residual,
                           delta=bf16_bits(delta), norm_w=bf16_bits(norm_w), eps=eps)
        want = O.gemv(w2.ravel(), vocab, cols, x)
        assert O.argmax(want) == rows_at[0]
        assert out["token"] == rows_at[0], f"ties at {rows_at}: got {out['token']}"
    for nan_at in (0, 4321, vocab - 1):
        w2 = w.reshape(vocab, cols).copy()
        w2[nan_at, 3] = np.nan
        out = K.gemv_fused(bf16_bits(w2.ravel()), vocab, cols, K.PRO_NORM, K.EPI_ARGMAX, f64, residual=residual,
                           delta=bf16_bits(delta), norm_w=bf16_bits(norm_w), eps=eps, advance=True, pos=3)
        assert np.isnan(out["y"][nan_at]) and out["token"] == NO_TOKEN, f"NaN at {nan_at}"
        assert out["pos"] == 4 and out["counter"] == 0


@pytest.mark.parametrize("f64", [False, True], ids=["f32", "f64"])
@pytest.mark.parametrize("cols", X_WIDTHS)
def test_the_plain_projection_is_the_gemv_at_every_model_width(K, cols, f64):
    """O's and down's instance (x given, bf16 out) and its f32-out twin, at the attention and MLP
    widths of Qwen3-0.6B/8B/32B (q_dim 2048/4096/8192 < 25600, intermediate 3072/12288/25600)."""
    for rows in (5, 1024 if cols > 5120 else 2053):
        rng = O.Rng(5000 + rows + cols)
        w = bf16s_with_edges(rng, rows * cols, 0.05)
        x = bf16s_with_edges(rng, cols, 1.0)
        want = O.gemv(w, rows, cols, x)
        mag = O.gemv_magnitude(w, rows, cols, x)
        for epi, rounded in ((K.EPI_BF16, True), (K.EPI_F32, False)):
            out = K.gemv_fused(bf16_bits(w), rows, cols, K.PRO_X, epi, f64, x=bf16_bits(x))
            what = f"gemv {rows}x{cols} {'bf16' if rounded else 'f32'} out, {'f64' if f64 else 'f32'} sums"
            got = bf16_vals(out["y"]) if rounded else out["y"]
            check_gemv(what, got, O.bf16_round(want) if (rounded and f64) else want, mag, rounded, f64)


def test_a_non_finite_input_reaches_only_the_rows_that_read_it(K):
    """A NaN weight makes its own row NaN and no other (gpu_kernels.rs:395-431), with f32 and f64
    sums."""
    rows, cols = 300, 4096
    rng = O.Rng(6000)
    w = rng.bf16s(rows * cols, 0.05).reshape(rows, cols)
    x = rng.bf16s(cols, 1.0)
    w[17, 100] = np.nan
    for f64 in (False, True):
        out = K.gemv_fused(bf16_bits(w.ravel()), rows, cols, K.PRO_X, K.EPI_F32, f64, x=bf16_bits(x))
        nan = np.isnan(out["y"])
        assert nan[17] and nan.sum() == 1


def test_refused_instances_and_buffers(K):
    """An instance the kernel does not build, a width past the staged x, or a missing buffer is a
    FormatError before any launch."""
    from x0ne_core import FormatError
    g = K.gpu
    with pytest.raises(FormatError):
        g.gemv_fused(w=16, y=16, x=16, rows=8, cols=64, prologue=0, epilogue=2)  # (X, SWIGLU)
    with pytest.raises(FormatError):
        g.gemv_fused(w=16, y=16, x=16, rows=8, cols=60, prologue=0, epilogue=0)  # cols % 8
    with pytest.raises(FormatError):
        g.gemv_fused(w=16, y=16, res_in=16, delta=16, norm_w=16, rows=8, cols=16392, prologue=1, epilogue=0)
    with pytest.raises(FormatError):
        g.gemv_fused(w=16, y=16, rows=8, cols=64, prologue=0, epilogue=0)  # no x
    with pytest.raises(FormatError):
        g.gemv_fused(w=24, y=16, x=16, rows=8, cols=64, prologue=0, epilogue=0)  # W misaligned
    with pytest.raises(FormatError):
        g.gemv_fused(w=16, y=16, res_in=16, delta=16, norm_w=16, rows=8, cols=64, prologue=1, epilogue=3)
    assert g.gemv_fused_blocks(w=16, y=16, x=16, rows=8, cols=64, prologue=0, epilogue=2) == 0


@pytest.mark.parametrize("cols", [8, 520, 4096])
def test_a_row_of_negative_zero_products_sums_to_negative_zero(K, cols):
    """The reference's f64 sums start from -0.0 (Rust's Iterator::sum, lib.rs:123-133): a row
    whose products are all -0.0 gives -0.0 (bf16 0x8000), a row with one +0.0 product gives +0.0,
    as the oracle does, in both accumulations and across the chunks past a narrow row (8 and 520
    columns pad to the tile)."""
    x = np.full(cols, -1.0, np.float32)
    x[1::2] = 2.0
    w = np.zeros((6, cols), np.float32)
    w[0, 1::2] = -0.0           # (+0)(-1) = -0 and (-0)(2) = -0: all -0
    w[1, 1::2] = -0.0
    w[1, 1] = 0.0               # one (+0)(2) = +0: +0
    w[3, 0::2] = -0.0           # (-0)(-1) = +0 everywhere: +0
    w[4, 1::2] = -0.0           # as row 0
    w[5, :] = 0.0
    w[5, 0] = 1.0               # a nonzero row: -1
    want = O.gemv(w.ravel(), 6, cols, x)
    for f64 in (False, True):
        out = K.gemv_fused(bf16_bits(w.ravel()), 6, cols, K.PRO_X, K.EPI_BF16, f64, x=bf16_bits(x))
        assert out["y"].tolist() == bf16_bits(want).tolist(), f"{'f64' if f64 else 'f32'} sums, {cols} columns"
    assert bf16_bits(want)[:5].tolist() == [0x8000, 0x0000, 0x0000, 0x0000, 0x8000]
