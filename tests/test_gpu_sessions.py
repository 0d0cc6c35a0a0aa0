"""Session semantics on the GPU: the counterpart of x0ne-core/oracle/tests/gpu_engine.rs:303-362
(a session with its cache is a recompute), :444-510 (a session after other requests is a session
on a fresh engine), :511-564 (client bytes are zero after every way out of a request), :566-632
(random sessions match a model of them), :634-720 (the edges of the context) and :771-854 (a
token whose embedding is not finite poisons its request only). The model is the CPU oracle's
forward with its own cache; tolerances are the model level's (gpu_engine.rs:29-32)."""
import numpy as np
import pytest

from common import O, reference_tensors, safetensors_bytes, tiny, wide
from test_gpu_engine import Fixture, assert_logits

pytestmark = pytest.mark.gpu


def scrubbed(e) -> bool:
    return e.client_data_is_zero() and e.host_buffers_are_zero()


def bits(row) -> np.ndarray:
    return np.asarray(row, np.float32).view(np.uint32).copy()


@pytest.mark.parametrize("which", [0, 1])
def test_a_session_with_its_cache_is_a_recompute(which):
    """After the prompt and after every step a session's logits are the oracle's with the same
    cache; a fresh session over the whole prefix (a recompute) gives the cached rows within the
    tolerance; and a session's first row has the bits of the greedy pass's last row."""
    f = [Fixture(tiny(2, 4, 2, False), 6), Fixture(wide(), 7)][which]
    e = f.engine(128)
    ids = f.tokens(15, 60)
    for split in [1, 2, 31, 59]:
        f.model.reset()
        want = f.model.extend(ids[:split])
        rows = []
        s = e.session(ids[:split])
        assert s.position() == split
        assert_logits(f"session after a prompt of {split}", s.logits(), want)
        for i, t in enumerate(ids[split:]):
            s.step(int(t))
            want = f.model.step(int(t))
            assert s.position() == split + i + 1
            assert_logits(f"session of {split}, step {i}", s.logits(), want)
            rows.append(s.logits())
        s.finish()
        assert scrubbed(e)
        for i in [0, len(rows) // 2, len(rows) - 1]:
            s = e.session(ids[:split + i + 1])
            assert_logits(f"cache of {split} + {i + 1} against a recompute", rows[i], s.logits())
            s.finish()
    tokens, last = e.greedy_with_last_logits(ids[:20], 1)
    s = e.session(ids[:20])
    assert (bits(s.logits()) == bits(last)).all(), "the session's first row is the greedy pass's"
    assert O.argmax(s.logits()) == int(tokens[0])
    s.finish()


def test_a_session_after_other_requests_is_a_session_on_a_fresh_engine():
    """Longer, shorter, abandoned, refused, greedy stopped early, both decode routes: each leaves
    nothing behind, so the same session afterwards has a new engine's bits."""
    from x0ne_core import DecodeMode, FormatError, Route
    f = Fixture(tiny(2, 4, 2, False), 10)
    prompt = f.tokens(20, 90)
    steps = f.tokens(21, 10)

    def run(e):
        s = e.session(prompt)
        rows = [bits(s.logits())]
        for t in steps:
            s.step(int(t))
            rows.append(bits(s.logits()))
        s.finish()
        return rows

    def same(a, b):
        return len(a) == len(b) and all((x == y).all() for x, y in zip(a, b))

    fresh = run(f.engine(600))
    e = f.engine(600)
    noise = f.tokens(22, 600)
    e.logits_at(noise, [599], Route.PREFILL)
    assert same(run(e), fresh), "after a long prefill"
    e.session(noise[:300])._drop()
    assert same(run(e), fresh), "after a session dropped without finish"
    s = e.session(noise[:5])
    s.step(1)
    with pytest.raises(FormatError):
        s.step(f.cfg.vocab)
    s._drop()
    assert same(run(e), fresh), "after a refused step"
    with pytest.raises(FormatError):
        e.session([f.cfg.vocab])
    with pytest.raises(FormatError):
        e.session([])
    assert same(run(e), fresh), "after refused sessions"
    g = e.session(noise[:40]).into_greedy(200)
    for _ in range(7):
        g.next_token()
    g._drop()
    assert same(run(e), fresh), "after a greedy session stopped early and dropped"
    e.logits_at(noise[:50], [49], Route.DECODE)
    e.set_decode_mode(DecodeMode.EAGER)
    e.logits_at(noise[:50], [49], Route.DECODE)
    e.set_decode_mode(DecodeMode.GRAPH)
    assert same(run(e), fresh), "after the decode routes"


def test_client_bytes_are_zero_after_every_way_out_of_a_request():
    """Finished, dropped, a greedy pass, a teacher-forced pass, refused requests, a greedy session
    dropped with steps in flight, an exception raised with a session open: the device's and the
    host's client bytes are zero after each, and the engine still serves."""
    from x0ne_core import Error, Route
    f = Fixture(tiny(2, 4, 2, False), 11)
    e = f.engine(128)
    assert scrubbed(e), "a new engine"
    ids = f.tokens(23, 100)
    s = e.session(ids)
    assert (s.logits() != 0).any()
    s.finish()
    assert scrubbed(e), "after finish"
    e.session(ids)._drop()
    assert scrubbed(e), "after a drop"
    e.greedy(ids, 20)
    assert scrubbed(e), "after a greedy pass"
    e.run(ids, Route.DECODE, keep=[3])
    assert scrubbed(e), "after a teacher-forced pass"
    with pytest.raises(Error):
        e.run(ids, Route.PREFILL, keep=[100])
    with pytest.raises(Error):
        e.greedy(ids, 30)  # 100 + 30 tokens in 128
    assert scrubbed(e), "after refused requests"
    g = e.session(ids[:10]).into_greedy(50)
    g.next_token()
    g._drop()
    assert scrubbed(e), "after a greedy session dropped with steps in flight"
    with pytest.raises(RuntimeError):
        with e.session(ids[:50]) as s:
            s.step(3)
            raise RuntimeError("the caller fails with a session open")
    assert scrubbed(e), "after an exception with a session open"
    s = e.session(ids[:50])
    f.model.reset()
    assert_logits("after every way out", s.logits(), f.model.logits(ids[:50])[49])
    s.finish()


def test_random_sessions_match_a_model_of_them():
    """Random operations on a session against the oracle with its cache: the position, the
    logits, a token outside the vocabulary refused without a change, a step in a full context
    refused without a change; then a random way out (finish, drop, or a greedy session asking
    more tokens than the context holds, refused); the client bytes are zero after each."""
    from x0ne_core import FormatError
    f = Fixture(tiny(2, 4, 2, False), 12)
    max_ctx = 48
    e = f.engine(max_ctx)
    vocab = f.cfg.vocab
    for seed in range(40):
        rng = O.Rng(1000 + seed)
        n = rng.pick([1, 2, 7, 40, 47, 48])
        prompt = rng.tokens(n, vocab)
        f.model.reset()
        want = f.model.extend(prompt)
        length = n
        s = e.session(prompt)
        for op in range(60):
            what = f"seed {seed} op {op} at {length}"
            assert s.position() == length, f"{what}: position"
            r = rng.below(8)
            if r == 0:
                bad = rng.pick([vocab, vocab + 1, 0xFFFFFFFF])
                before = bits(s.logits())
                with pytest.raises(FormatError):
                    s.step(bad)
                assert (bits(s.logits()) == before).all(), f"{what}: a refused step changed the logits"
            elif r == 1:
                assert_logits(what, s.logits(), want)
            else:
                t = rng.below(vocab)
                if length == max_ctx:
                    before = bits(s.logits())
                    with pytest.raises(FormatError):
                        s.step(t)
                    assert (bits(s.logits()) == before).all()
                else:
                    s.step(t)
                    want = f.model.step(t)
                    length += 1
        assert_logits(f"seed {seed}: at the end", s.logits(), want)
        way = rng.below(3)
        if way == 0:
            s.finish()
        elif way == 1:
            s._drop()
        else:
            with pytest.raises(FormatError):
                s.into_greedy(max_ctx - length + 2)
        assert scrubbed(e), f"seed {seed}: client bytes after the session"


def test_the_edges_of_the_context_are_served_and_bounded():
    """A prompt of one token, a prompt of the whole context, the last step that fits and the first
    that does not, the bounds of every entry point, and a context of one position."""
    from x0ne_core import Error, FormatError, GREEDY_AHEAD_MAX, Route
    f = Fixture(tiny(1, 2, 1, False), 13)
    full = f.cfg.max_pos
    e = f.engine(full)
    assert e.max_ctx() == full
    ids = f.tokens(24, full)
    want = f.model.logits(ids)
    assert_logits("a prompt of one token", e.logits_at(ids[:1], [0], Route.PREFILL)[0], want[0])
    assert_logits("a prompt of one token, decode", e.logits_at(ids[:1], [0], Route.DECODE)[0], want[0])
    assert e.greedy(ids[:1], 1).size == 1
    last = e.logits_at(ids, [full - 2, full - 1], Route.PREFILL)
    assert_logits("position max - 2", last[0], want[full - 2])
    assert_logits("position max - 1", last[1], want[full - 1])
    s = e.session(ids[:full - 3])
    for p in range(full - 3, full):
        s.step(int(ids[p]))
        assert_logits(f"stepped to {p}", s.logits(), want[p])
    assert s.position() == full
    with pytest.raises(FormatError):
        s.step(0)
    with pytest.raises(Error):
        s.into_greedy(2)
    g = e.session(ids).into_greedy(1)  # one token needs no step
    g._drop()
    e.session(ids).finish()
    longer = np.append(ids, 0)
    with pytest.raises(FormatError):
        e.session(longer)
    with pytest.raises(Error):
        e.logits_at(longer, [0], Route.PREFILL)
    assert e.greedy(ids, 1).size == 1, "the last position's argmax needs no step"
    with pytest.raises(Error):
        e.greedy(ids, 2)
    assert e.greedy(ids[:full - 9], 10).size == 10
    with pytest.raises(Error):
        e.greedy(ids[:full - 9], 11)
    with pytest.raises(Error):
        e.greedy(ids[:4], 0)
    with pytest.raises(Error):
        e.greedy([], 4)
    for ahead in [0, GREEDY_AHEAD_MAX + 1, 2 ** 63]:
        with pytest.raises(Error):
            e.session(ids[:4]).into_greedy_ahead(4, ahead)
    with pytest.raises(Error):
        e.session(ids[:4]).into_greedy(0)
    assert scrubbed(e)
    small = f.engine(1)
    assert_logits("max_ctx 1", small.logits_at(ids[:1], [0], Route.PREFILL)[0], want[0])
    with pytest.raises(Error):
        small.logits_at(ids[:2], [0], Route.PREFILL)
    s = small.session(ids[:1])
    with pytest.raises(Error):
        s.step(0)
    s.finish()


@pytest.mark.parametrize("special", [np.inf, np.nan], ids=["inf", "nan"])
def test_a_token_whose_embedding_is_not_finite_poisons_its_request_only(special):
    """A checkpoint with a non-finite value in token 7's embedding row: a request that feeds it has
    no finite logits from there on (the oracle says the same); its greedy pass and its
    teacher-forced pass are refused (GpuError: no argmax of a NaN row) and leave nothing; the
    positions before it are a request of their own; a session opens on it, steps, and cannot
    produce a greedy token; a clean request before and after gives the same bits."""
    from x0ne_core import Engine, EngineOptions, Error, GpuError, Route
    BAD = 7
    cfg = tiny(2, 4, 2, False)
    tensors = reference_tensors(cfg, 16)
    shape, emb = tensors["model.embed_tokens.weight"]
    emb = emb.copy()
    emb[BAD * cfg.hidden + 3] = O.bf16_bits(np.array([special], np.float32))[0]
    tensors["model.embed_tokens.weight"] = (shape, emb)
    model = O.Model(cfg, weights_bf16=True)
    for name, (_, b) in tensors.items():
        model.set(name, b)
    e = Engine.load_from(cfg.to_json(), {"model.safetensors": safetensors_bytes(tensors)},
                         EngineOptions(max_ctx=64, page_seed=7, f64_sums=False))
    clean = np.array([BAD + 1 if t == BAD else t for t in O.Rng(26).tokens(30, cfg.vocab)], np.uint32)
    before, row_before = e.greedy_with_last_logits(clean, 10)
    assert np.isfinite(row_before).all()
    dirty = clean.copy()
    dirty[12] = BAD
    with pytest.raises(GpuError):
        e.greedy(dirty, 5)
    assert scrubbed(e), "after the refused greedy pass"
    with pytest.raises(GpuError):
        e.logits_at(dirty, [11, 12, 29], Route.PREFILL)
    assert scrubbed(e), "after the refused pass"
    rows = e.logits_at(dirty[:12], [11], Route.PREFILL)
    assert np.isfinite(rows[0]).all(), "a position before the token"
    s = e.session(dirty[:13])
    assert np.isnan(s.logits()).all(), "the token's own position"
    s.finish()
    want = model.logits(dirty)
    assert np.isfinite(want[11]).all() and np.isnan(want[12]).all() and np.isnan(want[29]).all()
    s = e.session(dirty)
    assert np.isnan(s.logits()).all() and O.argmax(s.logits()) is None
    s.step(1)
    try:
        g = s.into_greedy(3)
        with pytest.raises(Error):
            g.next_token()
        g._drop()
    except Error:
        pass
    assert scrubbed(e), "after the poisoned session"
    after, row_after = e.greedy_with_last_logits(clean, 10)
    assert (before == after).all(), "the poisoned request changed a later one"
    assert (bits(row_before) == bits(row_after)).all()
