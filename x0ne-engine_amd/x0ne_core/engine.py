"""The engine (x0ne-core/runtime/src/engine.rs) over the C ABI: Engine, Session, Greedy.

Same names, argument meanings and error behaviour as the reference's Rust API: a Format error
comes before any device work; one Session at a time per Engine; a Session's logits are valid
until its next step or finish; a failed step ends the session's steps; finishing, dropping or
failing zeroes every client byte (device and host)."""
from __future__ import annotations

import ctypes as C
import json
import os
from dataclasses import dataclass
from enum import IntEnum

import numpy as np

from ._lib import Counts, EngineOptionsC, FormatError, PosStatsC, check, lib

GREEDY_AHEAD = 2  # engine.rs:78
GREEDY_AHEAD_MAX = 15  # engine.rs:73


class Route(IntEnum):
    PREFILL = 0
    DECODE = 1


class DecodeMode(IntEnum):
    EAGER = 0
    GRAPH = 1


class DecodeAttention(IntEnum):
    """ops.rs:55-62"""
    SPLIT_K = 0
    PER_HEAD = 1


class SplitMerge(IntEnum):
    """ops.rs:64-70"""
    KERNEL = 0
    LAST_BLOCK = 1


# x0ne_engine_options.sums
SUMS_DEFAULT, SUMS_F64, SUMS_F32 = 0, 1, 2


@dataclass
class EngineOptions:
    """EngineOptions (engine.rs:38-40) plus the KV page order (0: identity, else a seeded
    shuffle), the accumulation (f64_sums True: the exact mode, each exact product added in f64;
    False: the f32 path; None, the default: the exact mode wherever the engine can serve it,
    else f32), the prompt rows per prefill pass (0: min(2048, max_ctx)) and the sequences the
    batched greedy entry points serve (0 or 1: one)."""
    max_ctx: int
    page_seed: int = 0
    f64_sums: bool | None = None
    prefill_chunk: int = 0
    max_batch: int = 0

    def c(self):
        sums = SUMS_DEFAULT if self.f64_sums is None else SUMS_F64 if self.f64_sums else SUMS_F32
        return EngineOptionsC(self.max_ctx, self.page_seed, sums, int(self.prefill_chunk), int(self.max_batch), 0)


def _ids(ids):
    a = np.ascontiguousarray(ids, dtype=np.uint32)
    return a, a.ctypes.data_as(C.POINTER(C.c_uint32))


# PosStats (engine.rs:60-64).
POS_STATS = np.dtype([("argmax", np.uint32), ("logsumexp", np.float32), ("next_logprob", np.float32)])


class Engine:
    def __init__(self, handle, config: dict):
        self.h = handle
        self.config = config
        self._session = None

    @staticmethod
    def load_from(config_json, files: dict, opts: EngineOptions, index_json=None) -> "Engine":
        """Engine::load_from (engine.rs:301-309) over in-memory safetensors files {name: bytes}."""
        if isinstance(config_json, dict):
            config_json = json.dumps(config_json)
        names = list(files)
        blobs = [bytes(files[n]) for n in names]
        n = len(names)
        c_names = (C.c_char_p * max(1, n))(*[x.encode() for x in names])
        keep = [C.create_string_buffer(b, len(b)) for b in blobs]
        c_data = (C.c_void_p * max(1, n))(*[C.cast(k, C.c_void_p) for k in keep])
        c_lens = (C.c_uint64 * max(1, n))(*[len(b) for b in blobs])
        h = C.c_void_p()
        o = opts.c()
        idx = index_json.encode() if isinstance(index_json, str) else index_json
        check(lib().x0ne_engine_load_from(config_json.encode(), n, c_names, c_data, c_lens, idx, C.byref(o),
                                          C.byref(h)), "Engine::load_from")
        return Engine(h, json.loads(config_json))

    @staticmethod
    def load(model_dir, opts: EngineOptions) -> "Engine":
        """Engine::load (engine.rs:292-297): model_dir's config.json, then model.safetensors or the
        shards its model.safetensors.index.json names (Safetensors::open_dir, st.rs:158-181)."""
        h = C.c_void_p()
        o = opts.c()
        check(lib().x0ne_engine_load(os.fsencode(model_dir), C.byref(o), C.byref(h)), "Engine::load")
        e = Engine(h, {})  # freed on any error below
        with open(os.path.join(model_dir, "config.json"), encoding="utf-8") as f:
            e.config = json.loads(f.read())
        return e

    @staticmethod
    def load_synthetic(config_json, seed: int, std: float, opts: EngineOptions) -> "Engine":
        """This build's synthetic checkpoint: projections and embedding N(0, std) bf16 drawn on the
        device from `seed`, norm weights 1.0."""
        if isinstance(config_json, dict):
            config_json = json.dumps(config_json)
        h = C.c_void_p()
        o = opts.c()
        check(lib().x0ne_engine_load_synthetic(config_json.encode(), seed, float(std), C.byref(o), C.byref(h)),
              "Engine::load_synthetic")
        return Engine(h, json.loads(config_json))

    def close(self):
        if getattr(self, "h", None):
            if self._session is not None:
                self._session._drop()
            lib().x0ne_engine_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    # -- requests --
    def session(self, prompt) -> "Session":
        """Engine::session (engine.rs:389-406)."""
        a, p = _ids(prompt)
        h = C.c_void_p()
        check(lib().x0ne_engine_session(self.h, p, a.size, C.byref(h)), "session")
        s = Session(self, h)
        self._session = s
        return s

    def greedy_timed(self, prompt, n: int):
        """Engine::greedy_timed (engine.rs:1026-1038): tokens and per-token host times."""
        a, p = _ids(prompt)
        toks = np.zeros(n, np.uint32)
        times = np.zeros(n, np.float64)
        check(lib().x0ne_engine_greedy_timed(self.h, p, a.size, n, toks.ctypes.data_as(C.POINTER(C.c_uint32)),
                                             times.ctypes.data_as(C.POINTER(C.c_double))), "greedy")
        return toks, times

    def decode_timed(self, prompt, warmup: int, steps: int):
        """Prefill, `warmup` decode steps, then `steps` decode steps timed between two stream
        synchronisations: (tokens, seconds of the timed steps)."""
        a, p = _ids(prompt)
        toks = np.zeros(warmup + steps + 1, np.uint32)
        secs = C.c_double()
        check(lib().x0ne_engine_decode_timed(self.h, p, a.size, warmup, steps,
                                             toks.ctypes.data_as(C.POINTER(C.c_uint32)), C.byref(secs)),
              "decode_timed")
        return toks, secs.value

    def greedy(self, prompt, n: int) -> np.ndarray:
        return self.greedy_timed(prompt, n)[0]

    def greedy_batch(self, prompts, n: int, logits: bool = False):
        """Greedy decoding of independent prompts (rows of equal length) at once: tokens
        [batch][n], per-step host times, and with `logits` each sequence's last logits row."""
        a = np.ascontiguousarray(prompts, dtype=np.uint32)
        if a.ndim != 2:
            raise FormatError("prompts: one row per sequence")
        b, np_ = a.shape
        toks = np.zeros((b, n), np.uint32)
        times = np.zeros(n, np.float64)
        rows = np.zeros((b, self.vocab_size), np.float32) if logits else None
        check(lib().x0ne_engine_greedy_batch(
            self.h, a.ctypes.data_as(C.POINTER(C.c_uint32)), np_, b, n, toks.ctypes.data_as(C.POINTER(C.c_uint32)),
            times.ctypes.data_as(C.POINTER(C.c_double)),
            rows.ctypes.data_as(C.POINTER(C.c_float)) if logits else None), "greedy_batch")
        return (toks, times, rows) if logits else (toks, times)

    def decode_batch_timed(self, prompts, warmup: int, steps: int):
        """decode_timed for independent prompts at once: (tokens [batch][warmup + steps + 1],
        seconds of the timed steps)."""
        a = np.ascontiguousarray(prompts, dtype=np.uint32)
        b, np_ = a.shape
        toks = np.zeros((b, warmup + steps + 1), np.uint32)
        secs = C.c_double()
        check(lib().x0ne_engine_decode_batch_timed(self.h, a.ctypes.data_as(C.POINTER(C.c_uint32)), np_, b, warmup,
                                                   steps, toks.ctypes.data_as(C.POINTER(C.c_uint32)),
                                                   C.byref(secs)), "decode_batch_timed")
        return toks, secs.value

    def greedy_with_last_logits(self, prompt, n: int):
        a, p = _ids(prompt)
        toks = np.zeros(n, np.uint32)
        logits = np.zeros(self.vocab_size, np.float32)
        check(lib().x0ne_engine_greedy_with_last_logits(
            self.h, p, a.size, n, toks.ctypes.data_as(C.POINTER(C.c_uint32)),
            logits.ctypes.data_as(C.POINTER(C.c_float))), "greedy_with_last_logits")
        return toks, logits

    def logits_at(self, ids, positions, route: Route = Route.DECODE) -> list:
        """Engine::logits_at (engine.rs:1012-1020)."""
        a, p = _ids(ids)
        pos = np.ascontiguousarray(positions, np.uintp)
        rows = np.zeros((len(positions), self.vocab_size), np.float32)
        check(lib().x0ne_engine_logits_at(self.h, p, a.size, pos.ctypes.data_as(C.POINTER(C.c_size_t)), pos.size,
                                          int(route), rows.ctypes.data_as(C.POINTER(C.c_float))), "logits_at")
        return [rows[i] for i in range(len(positions))]

    def run(self, ids, route: Route = Route.DECODE, keep=()):
        """Engine::run (engine.rs:928-1006): per position (argmax, logsumexp, next_logprob) as a
        structured array, and the f32 logits rows at `keep`."""
        a, p = _ids(ids)
        kp = np.ascontiguousarray(keep, np.uintp)
        stats = (PosStatsC * max(1, a.size))()
        rows = np.zeros((kp.size, self.vocab_size), np.float32)
        check(lib().x0ne_engine_run(self.h, p, a.size, int(route), kp.ctypes.data_as(C.POINTER(C.c_size_t)), kp.size,
                                    stats, rows.ctypes.data_as(C.POINTER(C.c_float))), "run")
        out = np.zeros(a.size, POS_STATS)
        for i in range(a.size):
            out[i] = (stats[i].argmax, stats[i].logsumexp, stats[i].next_logprob)
        return out, [rows[i] for i in range(kp.size)]

    def moe_routing(self, ids) -> np.ndarray:
        """Engine::moe_routing (engine.rs:612-640): [position][layer][top_k] expert ids, flattened
        (empty for a dense engine)."""
        a, p = _ids(ids)
        c = self.config
        per = int(c.get("num_hidden_layers", 0)) * int(c.get("num_experts_per_tok", 0))
        out = np.zeros(max(1, a.size * per), np.uint32)
        n = C.c_size_t(0)
        check(lib().x0ne_engine_moe_routing(self.h, p, a.size, out.ctypes.data_as(C.POINTER(C.c_uint32)), out.size,
                                            C.byref(n)), "moe_routing")
        return out[:n.value].copy()

    def stats(self, ids, route: Route = Route.DECODE):
        """Engine::stats (engine.rs:1003-1006)."""
        return self.run(ids, route)[0]

    # -- introspection --
    @property
    def vocab_size(self) -> int:
        return int(self.config["vocab_size"])

    def describe(self) -> str:
        buf = C.create_string_buffer(2048)
        check(lib().x0ne_engine_describe(self.h, buf, 2048))
        return buf.value.decode()

    def set_decode_mode(self, mode: DecodeMode):
        check(lib().x0ne_engine_set_decode_mode(self.h, int(mode)), "set_decode_mode")

    def decode_mode(self) -> DecodeMode:
        return DecodeMode(lib().x0ne_engine_decode_mode(self.h))

    def set_decode_attention(self, a: DecodeAttention):
        """Engine::set_decode_attention (engine.rs:531-539): re-captures the decode graph, which
        zeroes the client buffers; call it between requests."""
        check(lib().x0ne_engine_set_decode_attention(self.h, int(a)), "set_decode_attention")

    def decode_attention(self) -> DecodeAttention:
        return DecodeAttention(lib().x0ne_engine_decode_attention(self.h))

    def set_split_merge(self, m: SplitMerge):
        """Engine::set_split_merge (engine.rs:547-560): LAST_BLOCK needs a grouped split-K kernel
        (GpuError otherwise); re-captures the decode graph."""
        check(lib().x0ne_engine_set_split_merge(self.h, int(m)), "set_split_merge")

    def split_merge(self) -> SplitMerge:
        return SplitMerge(lib().x0ne_engine_split_merge(self.h))

    def graph_nodes(self) -> int:
        return lib().x0ne_engine_graph_nodes(self.h)

    def splits(self) -> int:
        return lib().x0ne_engine_splits(self.h)

    def max_ctx(self) -> int:
        return lib().x0ne_engine_max_ctx(self.h)

    def exact(self) -> bool:
        """True when the engine runs the exact mode (f64 sums), the default resolved."""
        return lib().x0ne_engine_sums(self.h) == SUMS_F64

    def counts(self) -> dict:
        c = Counts()
        check(lib().x0ne_engine_counts(self.h, C.byref(c)))
        return c.as_dict()

    def client_data_is_zero(self) -> bool:
        out = C.c_int()
        check(lib().x0ne_engine_client_data_is_zero(self.h, C.byref(out)))
        return bool(out.value)

    def host_buffers_are_zero(self) -> bool:
        return bool(lib().x0ne_engine_host_buffers_are_zero(self.h))

    def arena(self):
        from .arena import Arena
        return Arena(lib().x0ne_engine_arena(self.h), owned=False)

    KERNELS = {"qkv": 0, "attention": 1, "o": 2, "gate_up": 3, "down": 4, "head": 5}

    def time_kernel(self, which: str, iters: int, batch: int = 0):
        """One decode-step kernel alone, `iters` rounds over every layer, launched back to back on
        the engine's stream: (average kernel duration in microseconds from the start/stop events
        hipExtLaunchKernel records, average wall time per launch with the gaps, launches).
        batch > 0: the batched step's kernel at that many sequences. The attention runs with
        every sequence at position max_ctx - 1."""
        kern, wall, n = C.c_double(), C.c_double(), C.c_uint64()
        if batch:
            check(lib().x0ne_engine_time_batch_kernel(self.h, self.KERNELS[which], batch, iters, C.byref(kern),
                                                      C.byref(wall), C.byref(n)), "time_batch_kernel")
        else:
            check(lib().x0ne_engine_time_kernel(self.h, self.KERNELS[which], iters, C.byref(kern), C.byref(wall),
                                                C.byref(n)), "time_kernel")
        return kern.value, wall.value, n.value

    def page(self, i: int) -> int:
        out = C.c_uint32()
        check(lib().x0ne_engine_page(self.h, i, C.byref(out)))
        return out.value


class Session:
    """A request on the engine (engine.rs:1137-1243)."""

    def __init__(self, engine: Engine, handle):
        self.e, self.h = engine, handle

    def _drop(self):
        if self.h:
            lib().x0ne_session_drop(self.h)
            self.h = None
            self.e._session = None

    def __del__(self):
        self._drop()

    # A `with` block is the scope a Rust Session lives in: leaving it by an exception drops the
    # session (zeroing the client bytes), as unwinding a panic drops it (engine.rs:1346-1353).
    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self._drop()
        return False

    def logits(self) -> np.ndarray:
        """f32 logits of the last position (a copy; empty after a failed step)."""
        ptr = C.POINTER(C.c_float)()
        n = C.c_size_t()
        check(lib().x0ne_session_logits(self.h, C.byref(ptr), C.byref(n)))
        if not ptr or n.value == 0:
            return np.zeros(0, np.float32)
        return np.ctypeslib.as_array(ptr, shape=(n.value,)).copy()

    def position(self) -> int:
        return lib().x0ne_session_position(self.h)

    def step(self, token: int):
        check(lib().x0ne_session_step(self.h, int(token) & 0xFFFFFFFF), "step")

    def finish(self):
        h, self.h = self.h, None
        self.e._session = None
        check(lib().x0ne_session_finish(h), "finish")

    def into_greedy(self, max_tokens: int) -> "Greedy":
        return self.into_greedy_ahead(max_tokens, GREEDY_AHEAD)

    def into_greedy_ahead(self, max_tokens: int, ahead: int) -> "Greedy":
        h, self.h = self.h, None
        self.e._session = None
        out = C.c_void_p()
        check(lib().x0ne_session_into_greedy(h, max_tokens, ahead, C.byref(out)), "into_greedy")
        g = Greedy(self.e, out)
        self.e._session = g
        return g


class Greedy:
    """A session decoding greedily on the device (engine.rs:1245-1344)."""

    def __init__(self, engine: Engine, handle):
        self.e, self.h = engine, handle

    def _drop(self):
        if self.h:
            lib().x0ne_greedy_drop(self.h)
            self.h = None
            self.e._session = None

    def __del__(self):
        self._drop()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self._drop()
        return False

    def next_token(self) -> int:
        out = C.c_uint32()
        check(lib().x0ne_greedy_next(self.h, C.byref(out)), "next_token")
        return out.value

    def taken(self) -> int:
        return lib().x0ne_greedy_taken(self.h)

    def position(self) -> int:
        return lib().x0ne_greedy_position(self.h)

    def finish(self):
        h, self.h = self.h, None
        self.e._session = None
        check(lib().x0ne_greedy_finish(h), "finish")
