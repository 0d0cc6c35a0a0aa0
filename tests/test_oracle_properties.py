"""The CPU oracle (oracle/) pinned where the reference's fixtures leave it open, without a GPU.

Each check is chosen so that a plausible mistake in the restatement fails it: bf16 rounding
exhaustively against a library routine that is round-to-nearest-even (torch's f32 -> bf16); the
kernels' closed forms and invariants (the properties the reference's own cpu_oracle.rs:35-447
checks); and brute force in numpy float64 on small inputs, written from the textbook definition.
"""
import math

import numpy as np
import pytest

from common import O, bf16_bits, bf16_vals

# ---------------------------------------------------------------------------------------------
# bf16 (oracle/src/bf16.rs:5-54)
# ---------------------------------------------------------------------------------------------


def test_bf16_rounding_is_round_to_nearest_even_against_torch():
    """Every upper half (sign, exponent, the 7 kept mantissa bits) with the lower halves that
    decide the rounding (0, 1, the tie 0x8000 and its neighbours, 0xFFFF) and 58 random ones:
    finite values and infinities round as torch's RNE conversion; a NaN keeps its sign and upper
    payload and gets the quiet bit 0x0040 (the reference's rule, where torch gives the canonical
    0x7FC0). X0NE_EXHAUSTIVE=1 runs all 2^32 patterns instead (about two minutes)."""
    import os
    import torch
    if os.environ.get("X0NE_EXHAUSTIVE") == "1":
        chunks = (np.arange(s, s + (1 << 26), dtype=np.uint64).astype(np.uint32) for s in range(0, 1 << 32, 1 << 26))
    else:
        lows = np.concatenate([[0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF],
                               np.random.default_rng(0).integers(0, 1 << 16, 58)]).astype(np.uint32)
        highs = np.arange(1 << 16, dtype=np.uint32) << 16
        chunks = [(highs[:, None] | lows[None, :]).ravel()]
    for u in chunks:
        f = u.view(np.float32)
        ours = bf16_bits(f)
        theirs = torch.from_numpy(f).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
        nan = np.isnan(f)
        assert (ours[~nan] == theirs[~nan]).all()
        assert (ours[nan] == ((u[nan] >> 16).astype(np.uint16) | 0x0040)).all()


def test_bf16_known_roundings_and_exact_decode():
    cases = [(1.0 + 2.0 ** -8, 0x3F80), (1.0 + 3 * 2.0 ** -8, 0x3F82), (1.0 + 2.0 ** -7, 0x3F81),
             (-(1.0 + 2.0 ** -8), 0xBF80), (0.0, 0x0000), (-0.0, 0x8000), (np.inf, 0x7F80), (-np.inf, 0xFF80)]
    for x, want in cases:
        assert int(bf16_bits(np.float32(x))[0]) == want, x
    # The largest finite f32 rounds past the largest bf16: infinity.
    assert int(bf16_bits(np.array([0x7F7FFFFF], np.uint32).view(np.float32))[0]) == 0x7F80
    # A denormal keeps its bits (no flush).
    assert int(bf16_bits(np.array([0x00010000], np.uint32).view(np.float32))[0]) == 0x0001
    every = np.arange(1 << 16, dtype=np.uint32)
    dec = bf16_vals(every.astype(np.uint16))
    assert (dec.view(np.uint32) == every << 16).all(), "decode is the bits shifted up"
    fin = np.isfinite(dec)
    assert (O.bf16_round(dec[fin]).view(np.uint32) == dec[fin].view(np.uint32)).all(), "idempotent"


# ---------------------------------------------------------------------------------------------
# Deterministic generator (this build's synthetic weights)
# ---------------------------------------------------------------------------------------------


def test_det_log_and_sincos_are_the_math_library_to_rounding():
    rng = np.random.default_rng(5)
    for x in np.concatenate([rng.uniform(1e-300, 1.0, 2000), [2.0 ** -53, 0.5, 1.0 - 2.0 ** -53, 1e-10]]):
        got, want = O.det_log(float(x)), math.log(float(x))
        assert abs(got - want) <= 4 * math.ulp(want), x
    for u in np.concatenate([rng.uniform(0.0, 1.0, 2000), [0.0, 0.25, 0.5, 0.75]]):
        s, c = O.det_sincos_turn(float(u))
        assert abs(s - math.sin(2 * math.pi * u)) <= 2e-15 and abs(c - math.cos(2 * math.pi * u)) <= 2e-15, u


def test_normal_draws_have_the_asked_moments_and_streams_differ():
    x = bf16_vals(O.normal_bf16(O.tensor_key(0, 3), 0, 1 << 20, 0.02)).astype(np.float64)
    assert abs(x.mean()) < 0.02 * 5 / 1024
    assert abs(x.std() / 0.02 - 1.0) < 5e-3
    # Tails: about 4.55 % beyond 2 sigma.
    assert abs((np.abs(x) > 0.04).mean() - 0.0455) < 0.002
    # A draw does not depend on where a read starts (the device fills in parallel chunks).
    key = O.tensor_key(0, 7)
    whole = O.normal_bf16(key, 0, 4096, 0.02)
    assert (O.normal_bf16(key, 1000, 96, 0.02) == whole[1000:1096]).all()
    keys = {O.tensor_key(0, i) for i in range(1000)} | {O.tensor_key(1, i) for i in range(1000)}
    assert len(keys) == 2000


# ---------------------------------------------------------------------------------------------
# Kernels (oracle/src/lib.rs:39-253)
# ---------------------------------------------------------------------------------------------


def test_embedding_copies_the_row_and_an_id_past_the_table_gives_zeros():
    table = np.arange(5 * 8, dtype=np.float32).reshape(5, 8)
    assert (O.embedding(table, 8, 3) == table[3]).all()
    assert (O.embedding(table, 8, 5) == 0).all() and (O.embedding(table, 8, 2 ** 32 - 1) == 0).all()


def test_add_rmsnorm_is_one_f32_add_then_unit_mean_square():
    rng = np.random.default_rng(1)
    for n in (8, 64, 4096):
        r = rng.normal(0, 3, n).astype(np.float32)
        x = rng.normal(0, 1, n).astype(np.float32)
        w = rng.uniform(0.5, 2, n).astype(np.float32)
        r_out, y = O.add_rmsnorm(r, x, w, 1e-6)
        assert (r_out.view(np.uint32) == (r + x).view(np.uint32)).all(), "one IEEE f32 add"
        rd = r_out.astype(np.float64)
        want = rd / np.sqrt(np.mean(rd * rd) + 1e-6) * w
        assert np.abs(y - want).max() <= 2e-7 * np.abs(want).max()
        # eps 0, unit weights: the mean square is 1 (a mean over n - 1, or a missing root, fails).
        _, y1 = O.add_rmsnorm(r, x, np.ones(n, np.float32), 0.0)
        assert abs(np.mean(y1.astype(np.float64) ** 2) - 1.0) < 1e-6


def test_inv_freq_is_the_f32_host_computation():
    for theta in (1e4, 1e6):
        i = np.arange(64, dtype=np.float32)
        want = np.float32(1.0) / np.power(np.float32(theta), i * np.float32(2) / np.float32(128))
        got = O.inv_freq_f32(128, theta)
        assert (np.abs(got.astype(np.float64) - want) <= 2 * np.spacing(want)).all()
        assert got[0] == 1.0


def rope_f64(x, w, inv, pos, eps):
    """Rotate-half RoPE after a per-head RMSNorm, as complex multiplication: pairs (i, i + 64)."""
    x = x.astype(np.float64)
    n = x / np.sqrt(np.mean(x * x) + eps) * w.astype(np.float64)
    z = (n[:64] + 1j * n[64:]) * np.exp(1j * (np.float32(pos) * inv).astype(np.float64))
    return np.concatenate([z.real, z.imag])


def test_qk_norm_rope_is_a_rotation_of_the_normed_head_and_v_passes():
    rng = np.random.default_rng(2)
    qh, kvh = 4, 2
    inv = O.inv_freq_f32(128, 1e6)
    qkv = rng.normal(0, 2, (qh + 2 * kvh) * 128).astype(np.float32)
    qn, kn = rng.uniform(0.5, 1.5, 128).astype(np.float32), rng.uniform(0.5, 1.5, 128).astype(np.float32)
    for pos in (0, 1, 17, 4095, 40959):
        q, k, v = O.qk_norm_rope(qkv, qn, kn, inv, qh, kvh, 128, pos, 1e-6)
        assert (v == qkv[(qh + kvh) * 128:]).all()
        for h in range(qh):
            want = rope_f64(qkv[h * 128:(h + 1) * 128], qn, inv, pos, 1e-6)
            assert np.abs(q[h * 128:(h + 1) * 128] - want).max() <= 1e-6 * np.abs(want).max()
        for h in range(kvh):
            want = rope_f64(qkv[(qh + h) * 128:(qh + h + 1) * 128], kn, inv, pos, 1e-6)
            assert np.abs(k[h * 128:(h + 1) * 128] - want).max() <= 1e-6 * np.abs(want).max()
        # The rotation keeps each pair's length.
        q0, _, _ = O.qk_norm_rope(qkv, qn, kn, inv, qh, kvh, 128, 0, 1e-6)
        l0 = q0[:64].astype(np.float64) ** 2 + q0[64:128].astype(np.float64) ** 2
        lp = q[:64].astype(np.float64) ** 2 + q[64:128].astype(np.float64) ** 2
        assert np.abs(lp - l0).max() <= 1e-5 * l0.max()


def attention_f64(q, k, v, ctx, qh, kvh):
    out = np.empty(qh * 128)
    g = qh // kvh
    k = k[:ctx * kvh * 128].astype(np.float64).reshape(ctx, kvh, 128)
    v = v[:ctx * kvh * 128].astype(np.float64).reshape(ctx, kvh, 128)
    for h in range(qh):
        s = k[:, h // g, :] @ q[h * 128:(h + 1) * 128].astype(np.float64) / math.sqrt(128)
        p = np.exp(s - s.max())
        out[h * 128:(h + 1) * 128] = (p / p.sum()) @ v[:, h // g, :]
    return out


def test_attention_is_softmax_attention_with_gqa_heads():
    rng = np.random.default_rng(3)
    for qh, kvh in ((1, 1), (4, 2), (8, 2)):
        for ctx in (1, 2, 7, 40):
            q = rng.normal(0, 1, qh * 128).astype(np.float32)
            k = rng.normal(0, 1, ctx * kvh * 128).astype(np.float32)
            v = rng.normal(0, 1, ctx * kvh * 128).astype(np.float32)
            got = O.attention_decode(q, k, v, ctx, qh, kvh)
            want = attention_f64(q, k, v, ctx, qh, kvh)
            assert np.abs(got - want).max() <= 1e-6 * np.abs(want).max() + 1e-12, (qh, kvh, ctx)
            vv = v.reshape(ctx, kvh, 128)
            for h in range(qh):  # each output stays in the hull of its kv head's values
                lo, hi = vv[:, h // (qh // kvh), :].min(0), vv[:, h // (qh // kvh), :].max(0)
                o = got[h * 128:(h + 1) * 128]
                assert (o >= lo - 1e-5).all() and (o <= hi + 1e-5).all()


def test_attention_one_key_gives_its_value_and_order_does_not_matter():
    rng = np.random.default_rng(4)
    qh, kvh, ctx = 4, 2, 9
    q = rng.normal(0, 1, qh * 128).astype(np.float32)
    k = rng.normal(0, 1, ctx * kvh * 128).astype(np.float32)
    v = rng.normal(0, 1, ctx * kvh * 128).astype(np.float32)
    one = O.attention_decode(q, k, v, 1, qh, kvh)
    for h in range(qh):
        assert (one[h * 128:(h + 1) * 128] == v[(h // 2) * 128:(h // 2 + 1) * 128]).all()
    perm = rng.permutation(ctx)
    kp = k.reshape(ctx, -1)[perm].ravel()
    vp = v.reshape(ctx, -1)[perm].ravel()
    a, b = O.attention_decode(q, k, v, ctx, qh, kvh), O.attention_decode(q, kp, vp, ctx, qh, kvh)
    assert np.abs(a - b).max() <= 1e-6
    # Adding the same vector to every key shifts every score of a head alike: no change.
    shift = np.tile(rng.normal(0, 1, kvh * 128).astype(np.float32), ctx)
    c = O.attention_decode(q, (k.astype(np.float64) + shift).astype(np.float32), v, ctx, qh, kvh)
    assert np.abs(a - c).max() <= 1e-4


def test_swiglu_special_values_and_formula():
    g = np.array([0.0, 1.0, -1.0, 30.0, -30.0, 2.5, np.nan, 1.0], np.float32)
    u = np.array([3.0, 2.0, 2.0, 1.0, 1.0, 0.0, 1.0, np.nan], np.float32)
    got = O.swiglu(np.concatenate([g, u]))
    gd, ud = g.astype(np.float64), u.astype(np.float64)
    want = gd / (1 + np.exp(-gd)) * ud
    fin = np.isfinite(want)
    assert (np.abs(got[fin] - want[fin]) <= 1e-7 * np.abs(want[fin]) + 1e-30).all()
    assert got[0] == 0.0 and got[5] == 0.0 and np.isnan(got[6]) and np.isnan(got[7])
    assert abs(got[3] - 30.0) < 1e-5 and abs(got[4]) < 1e-11


def test_argmax_takes_the_first_largest_and_a_nan_row_has_none():
    assert O.argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert O.argmax([-np.inf, -np.inf]) == 0
    assert O.argmax([1.0, np.nan, 5.0]) is None
    assert O.argmax(np.array([], np.float32)) is None
    assert O.argmax([np.inf, 1.0, np.inf]) == 0


def test_logsumexp_and_kl_hand_computed():
    assert abs(O.logsumexp([0.0, 0.0]) - math.log(2)) < 1e-12
    assert abs(O.logsumexp([1000.0, 1000.0]) - (1000 + math.log(2))) < 1e-9
    p = np.array([0.0, math.log(3)], np.float32)  # probabilities 1/4, 3/4
    q = np.array([0.0, 0.0], np.float32)          # 1/2, 1/2
    pp = np.array([0.25, 0.75])
    want = float((pp * np.log(pp / 0.5)).sum())
    assert abs(O.kl(p, q) - want) < 1e-7
    assert O.kl(p, p) == 0.0


def test_gemv_is_an_f64_dot_product_rounded_once():
    rng = np.random.default_rng(6)
    for rows, cols in ((1, 8), (7, 64), (33, 1000)):
        w = O.bf16_round(rng.normal(0, 1, rows * cols).astype(np.float32))
        x = O.bf16_round(rng.normal(0, 1, cols).astype(np.float32))
        want = (w.reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)).astype(np.float32)
        got = O.gemv(w, rows, cols, x)
        assert (np.abs(got - want) <= np.spacing(np.abs(want))).all()
        assert (O.gemv(bf16_bits(w).reshape(-1), rows, cols, x) == got).all(), "bf16 weights: same bits"


# ---------------------------------------------------------------------------------------------
# The forward (oracle/src/model.rs)
# ---------------------------------------------------------------------------------------------


def small_model(seed=0, tied=False):
    cfg = O.Config(64, 96, 2, 4, 2, 128, 300, 512, eps=1e-6, theta=1e6, tied=tied)
    m = O.Model(cfg, weights_bf16=True)
    m.init_normal(seed, 0.5)
    return cfg, m


def test_the_cache_gives_the_recompute_bit_for_bit():
    """Step by step through the cache equals the whole sequence at once (cpu_oracle.rs:502-565)."""
    cfg, m = small_model()
    ids = O.Rng(9).tokens(23, cfg.vocab)
    m.reset()
    whole = np.array(m.logits(ids))
    m.reset()
    stepped = [m.step(int(t)) for t in ids]
    assert (np.array(stepped).view(np.uint32) == whole.view(np.uint32)).all()
    # Truncating the cache and stepping again gives the same rows.
    m.truncate(10)
    again = [m.step(int(t)) for t in ids[10:]]
    assert (np.array(again).view(np.uint32) == whole[10:].view(np.uint32)).all()


def test_greedy_is_argmax_of_the_logits_it_stepped():
    cfg, m = small_model(1)
    prompt = O.Rng(3).tokens(5, cfg.vocab)
    toks, margins = m.greedy(prompt, 12)
    m.reset()
    seq = np.concatenate([prompt, toks[:-1]])
    rows = np.array(m.logits(seq))[len(prompt) - 1:]
    assert [O.argmax(r) for r in rows] == toks.tolist()
    s = np.sort(rows, axis=1)
    assert np.allclose(s[:, -1] - s[:, -2], margins)


def test_the_reference_routing_chooses_the_largest_and_normalises():
    """cpu_oracle.rs:449-498: per row the chosen experts are the largest, in order (larger logit,
    then the smaller index), distinct, none left out larger than the last; the weights a
    decreasing distribution; a row with a non-finite logit has no expert and NaN weights; an
    expert outside the table gives a NaN row and the others are their GEMV; the combination by
    hand."""
    rng = O.Rng(9)
    for _ in range(2000):
        experts = rng.range(1, 24)
        top_k = rng.range(1, experts)
        row = (np.array([float(rng.below(3)) for _ in range(experts)], np.float32) if rng.chance(3)
               else np.asarray(rng.f32s(experts, 8.0), np.float32))
        poisoned = rng.chance(8)
        if poisoned:
            row[rng.below(experts)] = rng.pick([np.nan, np.inf, -np.inf])
        ids, w = O.moe_route(row, experts, top_k)
        assert ids.size == top_k and w.size == top_k
        if poisoned:
            assert (ids == O.MOE_NO_EXPERT).all() and np.isnan(w).all()
            continue
        for a, b in zip(ids[:-1], ids[1:]):
            assert row[a] > row[b] or (row[a] == row[b] and a < b), (row, ids)
        assert len(set(ids.tolist())) == top_k
        least = row[ids[-1]]
        assert all(row[i] <= least for i in range(experts) if i not in set(ids.tolist()))
        assert abs(float(np.sum(w.astype(np.float64))) - 1.0) < 1e-6
        assert (w[:-1] >= w[1:]).all() and ((w > 0).all() or top_k > 1)
    w = np.asarray(rng.bf16s(3 * 4 * 8, 1.0), np.float32)
    x = np.asarray(rng.bf16s(2 * 8, 1.0), np.float32)
    y = O.moe_gemv(w, 3, 4, 8, [2, 3, O.MOE_NO_EXPERT, 0], x, 2)
    assert (y[:4] == O.gemv(w[2 * 32:], 4, 8, x[:8])).all()
    assert np.isnan(y[4:12]).all()
    assert (y[12:] == O.gemv(w[:32], 4, 8, x[8:])).all()
    assert O.moe_combine([1.0, 2.0, 3.0, 4.0], [0.25, 0.75], 2, 2).tolist() == [2.5, 3.5]


def test_routing_ties_keep_the_smaller_index_and_signed_zeros_are_equal():
    """The stable order of the reference (lib.rs:268-270): equal logits, -0.0 and 0.0 among them,
    keep the smaller index first; the weights of equal logits are equal."""
    ids, w = O.moe_route(np.array([0.0, -0.0, 1.0, 1.0, -0.0], np.float32), 5, 4)
    assert ids.tolist() == [2, 3, 0, 1]
    assert w[0] == w[1] and w[2] == w[3] and w[0] > w[2]


def test_the_oracles_sums_start_from_negative_zero_as_rusts_sum_does():
    """Iterator::sum::<f64>() folds from -0.0 in the Rust the reference pins (1.98.1): a GEMV row
    whose products are all negative zeros sums to -0.0, one with a positive zero among them to
    +0.0 (lib.rs:123-133); the same for the expert combination (lib.rs:314-329). The attention's
    output starts from an explicit 0f64 (lib.rs:167): a V column of negative zeros gives +0.0."""
    neg = np.float32(-0.0).view(np.uint32)
    pos = np.float32(0.0).view(np.uint32)
    w = np.array([0.0, -0.0, 0.0, 0.0, 0.0, 0.0], np.float32)
    y = O.gemv(w, 3, 2, np.array([-1.0, 1.0], np.float32))
    # rows: (+0 * -1, -0 * 1) = (-0, -0); (+0 * -1, +0 * 1) = (-0, +0); the same again
    assert y.view(np.uint32).tolist() == [neg, pos, pos]
    y4 = O.gemv(np.zeros(4 * 3, np.float32), 4, 3, np.array([-1.0, -2.0, -3.0], np.float32))
    assert (y4.view(np.uint32) == neg).all(), "every row of a 4-row block"
    c = O.moe_combine(np.array([-0.0, -0.0], np.float32), np.array([1.0, 0.5], np.float32), 1, 2)
    assert c.view(np.uint32).tolist() == [neg]
    q = np.ones(128, np.float32)
    k = np.ones(2 * 128, np.float32)
    v = np.full(2 * 128, -0.0, np.float32)
    out = O.attention_decode(q, k, v, 2, 1, 1)
    assert (np.asarray(out, np.float32).view(np.uint32) == pos).all()
