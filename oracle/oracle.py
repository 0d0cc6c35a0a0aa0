"""ctypes view of the CPU oracle (liboracle.so), for tests, smoke() and bench.py's cpu_baseline.

TEST INFRASTRUCTURE, NOT PRODUCT: the GPU path never imports this module. Every function here
is a thin call into x0ne_oracle.c, which restates x0ne-core/oracle/src/{bf16,lib,model}.rs.
Arrays are numpy: f32 values of bf16 where the reference passes f32 (lib.rs:4-7), or uint16
bf16 bit patterns where noted.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# X0NE_ORACLE_LIB: another build of the same restatement (the Makefile's sanitizer build).
LIB_PATH = os.environ.get("X0NE_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")

_lib = None


def build(force: bool = False) -> str:
    """Compiles liboracle.so with the Makefile beside this file."""
    cmd = ["make", "-C", HERE] + (["-B"] if force else [])
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


F32P = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
F64P = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
U16P = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
U32P = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")


class XoConfig(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32),
        ("inter", C.c_uint32),
        ("layers", C.c_uint32),
        ("q_heads", C.c_uint32),
        ("kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("vocab", C.c_uint32),
        ("max_pos", C.c_uint32),
        ("eps", C.c_float),
        ("tied", C.c_uint32),
        ("round_bf16", C.c_uint32),
    ]


def _declare(L):
    S = C.c_size_t
    L.xo_bf16_bits.argtypes = [C.c_float]
    L.xo_bf16_bits.restype = C.c_uint16
    L.xo_bf16_value.argtypes = [C.c_uint16]
    L.xo_bf16_value.restype = C.c_float
    L.xo_bf16_round.argtypes = [C.c_float]
    L.xo_bf16_round.restype = C.c_float
    L.xo_bf16_round_all.argtypes = [F32P, S]
    L.xo_bf16_encode.argtypes = [F32P, U16P, S]
    L.xo_bf16_decode.argtypes = [U16P, F32P, S]
    L.xo_bf16_ulp.argtypes = [C.c_float]
    L.xo_bf16_ulp.restype = C.c_double
    L.xo_rng_next.argtypes = [C.POINTER(C.c_uint64)]
    L.xo_rng_next.restype = C.c_uint64
    L.xo_rng_unit.argtypes = [C.POINTER(C.c_uint64)]
    L.xo_rng_unit.restype = C.c_float
    L.xo_rng_tokens.argtypes = [C.POINTER(C.c_uint64), U32P, S, C.c_uint64]
    L.xo_rng_bf16s.argtypes = [C.POINTER(C.c_uint64), F32P, S, C.c_float]
    L.xo_det_log.argtypes = [C.c_double]
    L.xo_det_log.restype = C.c_double
    L.xo_det_sincos_turn.argtypes = [C.c_double, C.POINTER(C.c_double), C.POINTER(C.c_double)]
    L.xo_normal_at.argtypes = [C.c_uint64, C.c_uint64]
    L.xo_normal_at.restype = C.c_double
    L.xo_normal_bf16.argtypes = [C.c_uint64, C.c_uint64, S, C.c_double, U16P]
    L.xo_tensor_key.argtypes = [C.c_uint64, C.c_uint64]
    L.xo_tensor_key.restype = C.c_uint64
    L.xo_set_threads.argtypes = [C.c_int]
    L.xo_threads.restype = C.c_int
    L.xo_embedding.argtypes = [F32P, S, S, C.c_uint32, F32P]
    L.xo_add_rmsnorm.argtypes = [F32P, F32P, F32P, S, C.c_float, F32P]
    L.xo_inv_freq_f64.argtypes = [S, C.c_double, F64P]
    L.xo_inv_freq_f32.argtypes = [S, C.c_float, F32P]
    L.xo_attn_scale.argtypes = [S]
    L.xo_attn_scale.restype = C.c_float
    L.xo_qk_norm_rope.argtypes = [F32P, F32P, F32P, F32P, S, S, S, C.c_uint32, C.c_float,
                                  F32P, F32P, F32P]
    L.xo_gemv.argtypes = [F32P, S, S, F32P, F32P]
    L.xo_gemv_bf16w.argtypes = [U16P, S, S, F32P, F32P]
    L.xo_gemv_magnitude.argtypes = [F32P, S, S, F32P, F64P]
    L.xo_attention_decode.argtypes = [F32P, F32P, F32P, S, S, S, S, F32P]
    L.xo_swiglu.argtypes = [F32P, S, F32P]
    L.xo_moe_route.argtypes = [F32P, S, S, S, U32P, F32P]
    L.xo_moe_gemv.argtypes = [F32P, S, S, S, U32P, S, F32P, S, F32P]
    L.xo_moe_combine.argtypes = [F32P, F32P, S, S, S, F32P]
    L.xo_argmax.argtypes = [F32P, S]
    L.xo_argmax.restype = C.c_int64
    L.xo_logsumexp.argtypes = [F32P, S]
    L.xo_logsumexp.restype = C.c_double
    L.xo_kl.argtypes = [F32P, F32P, S]
    L.xo_kl.restype = C.c_double
    L.xo_model_new.argtypes = [C.POINTER(XoConfig), F32P, C.c_int]
    L.xo_model_new.restype = C.c_void_p
    L.xo_model_free.argtypes = [C.c_void_p]
    L.xo_tensor_count.argtypes = [C.POINTER(XoConfig)]
    L.xo_tensor_count.restype = S
    L.xo_tensor_info.argtypes = [C.POINTER(XoConfig), S, C.c_char_p, S]
    L.xo_tensor_info.restype = S
    L.xo_model_set.argtypes = [C.c_void_p, S, S, C.c_void_p, S]
    L.xo_model_set.restype = C.c_int
    L.xo_model_init_normal.argtypes = [C.c_void_p, C.c_uint64, C.c_double]
    L.xo_model_init_normal.restype = C.c_int
    L.xo_model_init_reference.argtypes = [C.c_void_p, C.c_uint64]
    L.xo_model_init_reference.restype = C.c_int
    L.xo_model_reset.argtypes = [C.c_void_p]
    L.xo_model_len.argtypes = [C.c_void_p]
    L.xo_model_len.restype = S
    L.xo_model_truncate.argtypes = [C.c_void_p, S]
    L.xo_model_step.argtypes = [C.c_void_p, C.c_uint32, F32P]
    L.xo_model_step.restype = C.c_int
    L.xo_model_cache_row.argtypes = [C.c_void_p, S, S, F32P, F32P]
    L.xo_model_cache_row.restype = C.c_int
    L.xo_model_greedy.argtypes = [C.c_void_p, U32P, S, S, U32P, F32P]
    L.xo_model_greedy.restype = S


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- bf16 (bf16.rs) ----

def bf16_bits(x) -> np.ndarray:
    x = f32(np.atleast_1d(x))
    out = np.empty(x.shape, np.uint16)
    lib().xo_bf16_encode(x.ravel(), out.ravel(), x.size)
    return out


def bf16_values(bits) -> np.ndarray:
    b = np.ascontiguousarray(np.atleast_1d(bits), dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().xo_bf16_decode(b.ravel(), out.ravel(), b.size)
    return out


def bf16_round(x) -> np.ndarray:
    x = f32(np.array(x, dtype=np.float32, copy=True))
    lib().xo_bf16_round_all(x.ravel(), x.size)
    return x


def bf16_ulp(x: float) -> float:
    return lib().xo_bf16_ulp(float(x))


# ---- splitmix64 (common/mod.rs:8-53) ----

class Rng:
    """The reference tests' splitmix64 generator, stepping the C state."""

    def __init__(self, seed: int):
        self.state = C.c_uint64(seed & (2**64 - 1))

    def next_u64(self) -> int:
        return lib().xo_rng_next(C.byref(self.state))

    def below(self, n: int) -> int:
        return self.next_u64() % n

    def range(self, lo: int, hi: int) -> int:
        return lo + self.below(hi - lo + 1)

    def chance(self, one_in: int) -> bool:
        return self.below(one_in) == 0

    def pick(self, of):
        return of[self.below(len(of))]

    def unit(self) -> float:
        return lib().xo_rng_unit(C.byref(self.state))

    def f32s(self, n: int, scale: float) -> np.ndarray:
        return np.array([self.unit() * np.float32(scale) for _ in range(n)], np.float32) \
            if n < 64 else self._f32s_fast(n, scale)

    def _f32s_fast(self, n, scale):
        out = np.empty(n, np.float32)
        for i in range(n):
            out[i] = np.float32(self.unit()) * np.float32(scale)
        return out

    def bf16s(self, n: int, scale: float) -> np.ndarray:
        out = np.empty(n, np.float32)
        lib().xo_rng_bf16s(C.byref(self.state), out, n, float(scale))
        return out

    def tokens(self, n: int, vocab: int) -> np.ndarray:
        out = np.empty(n, np.uint32)
        lib().xo_rng_tokens(C.byref(self.state), out, n, vocab)
        return out


def synthetic_ids(n: int, vocab: int, seed: int) -> np.ndarray:
    return Rng(seed).tokens(n, vocab)


# ---- deterministic normal generator ----

def normal_at(key: int, i: int) -> float:
    return lib().xo_normal_at(key, i)


def normal_bf16(key: int, first: int, n: int, std: float) -> np.ndarray:
    out = np.empty(n, np.uint16)
    lib().xo_normal_bf16(key, first, n, std, out)
    return out


def tensor_key(seed: int, index: int) -> int:
    return lib().xo_tensor_key(seed, index)


def det_log(x: float) -> float:
    return lib().xo_det_log(x)


def det_sincos_turn(u: float):
    s, c = C.c_double(), C.c_double()
    lib().xo_det_sincos_turn(u, C.byref(s), C.byref(c))
    return s.value, c.value


def set_threads(n: int):
    lib().xo_set_threads(int(n))


def threads() -> int:
    return lib().xo_threads()


# ---- kernels (lib.rs) ----

def embedding(table: np.ndarray, hidden: int, token: int) -> np.ndarray:
    table = f32(table).ravel()
    out = np.empty(hidden, np.float32)
    lib().xo_embedding(table, table.size // hidden, hidden, token & 0xFFFFFFFF, out)
    return out


def add_rmsnorm(residual: np.ndarray, x, w, eps: float):
    """Returns (residual after the f32 add, normed row unrounded)."""
    r = f32(np.array(residual, np.float32, copy=True))
    x, w = f32(x), f32(w)
    out = np.empty(r.size, np.float32)
    lib().xo_add_rmsnorm(r, x, w, r.size, eps, out)
    return r, out


def inv_freq_f32(head_dim: int, theta: float) -> np.ndarray:
    out = np.empty(head_dim // 2, np.float32)
    lib().xo_inv_freq_f32(head_dim, theta, out)
    return out


def inv_freq_f64(head_dim: int, theta: float) -> np.ndarray:
    out = np.empty(head_dim // 2, np.float64)
    lib().xo_inv_freq_f64(head_dim, theta, out)
    return out


def attn_scale(head_dim: int) -> float:
    return lib().xo_attn_scale(head_dim)


def qk_norm_rope(qkv, q_norm, k_norm, inv_freq, q_heads, kv_heads, head_dim, pos, eps):
    qkv, qn, kn, inv = f32(qkv), f32(q_norm), f32(k_norm), f32(inv_freq)
    q = np.empty(q_heads * head_dim, np.float32)
    k = np.empty(kv_heads * head_dim, np.float32)
    v = np.empty(kv_heads * head_dim, np.float32)
    lib().xo_qk_norm_rope(qkv, qn, kn, inv, q_heads, kv_heads, head_dim, pos, eps, q, k, v)
    return q, k, v


MOE_NO_EXPERT = 0xFFFFFFFF


def moe_route(logits, experts: int, top_k: int):
    """lib.rs:254-282: (ids [rows][top_k] u32, weights [rows][top_k] f32), flattened."""
    lg = f32(logits).ravel()
    assert experts > 0 and 0 < top_k <= experts and top_k <= 64 and lg.size % experts == 0
    rows = lg.size // experts
    ids = np.empty(rows * top_k, np.uint32)
    w = np.empty(rows * top_k, np.float32)
    lib().xo_moe_route(lg, rows, experts, top_k, ids, w)
    return ids, w


def moe_gemv(w, experts: int, rows: int, cols: int, ids, x, x_group: int) -> np.ndarray:
    """lib.rs:284-312: [slots][rows] f32, flattened."""
    wf, xf = f32(w).ravel(), f32(x).ravel()
    ids = np.ascontiguousarray(ids, np.uint32)
    assert wf.size == experts * rows * cols and x_group > 0 and xf.size == ids.size // x_group * cols
    y = np.empty(ids.size * rows, np.float32)
    lib().xo_moe_gemv(wf, experts, rows, cols, ids, ids.size, xf, x_group, y)
    return y


def moe_combine(y, weights, hidden: int, top_k: int) -> np.ndarray:
    """lib.rs:314-329: [rows][hidden] f32, flattened."""
    yf, wf = f32(y).ravel(), f32(weights).ravel()
    assert wf.size % top_k == 0 and yf.size == wf.size * hidden
    rows = wf.size // top_k
    out = np.empty(rows * hidden, np.float32)
    lib().xo_moe_combine(yf, wf, rows, hidden, top_k, out)
    return out


def gemv(w: np.ndarray, rows: int, cols: int, x) -> np.ndarray:
    y = np.empty(rows, np.float32)
    if w.dtype == np.uint16:
        lib().xo_gemv_bf16w(np.ascontiguousarray(w).ravel(), rows, cols, f32(x), y)
    else:
        lib().xo_gemv(f32(w).ravel(), rows, cols, f32(x), y)
    return y


def gemv_magnitude(w, rows, cols, x) -> np.ndarray:
    y = np.empty(rows, np.float64)
    lib().xo_gemv_magnitude(f32(w).ravel(), rows, cols, f32(x), y)
    return y


def attention_decode(q, k, v, ctx, q_heads, kv_heads, head_dim=128) -> np.ndarray:
    q, k, v = f32(q).ravel(), f32(k).ravel(), f32(v).ravel()
    out = np.empty(q_heads * head_dim, np.float32)
    lib().xo_attention_decode(q, k, v, ctx, q_heads, kv_heads, head_dim, out)
    return out


def attention_rows(q, k, v, pos0, q_heads, kv_heads, head_dim, rows):
    """lib.rs:189-201: row r of q sits at pos0 + r and reads keys 0..=pos0 + r."""
    qd = q_heads * head_dim
    q = f32(q).ravel()
    return [attention_decode(q[r * qd:(r + 1) * qd], k, v, pos0 + r + 1, q_heads, kv_heads,
                             head_dim) for r in rows]


def swiglu(gate_up) -> np.ndarray:
    gu = f32(gate_up)
    out = np.empty(gu.size // 2, np.float32)
    lib().xo_swiglu(gu, gu.size // 2, out)
    return out


def argmax(x):
    x = f32(x)
    r = lib().xo_argmax(x, x.size)
    return None if r < 0 else int(r)


def logsumexp(x) -> float:
    x = f32(x)
    return lib().xo_logsumexp(x, x.size)


def kl(p, q) -> float:
    p, q = f32(p), f32(q)
    return lib().xo_kl(p, q, p.size)


# ---- the forward (model.rs) ----

class Config:
    """model.rs:12-26, with the rounding switch of this restatement."""

    def __init__(self, hidden, inter, layers, q_heads, kv_heads, head_dim, vocab, max_pos,
                 eps=1e-6, theta=1e6, tied=False, round_bf16=True):
        self.hidden, self.inter, self.layers = hidden, inter, layers
        self.q_heads, self.kv_heads, self.head_dim = q_heads, kv_heads, head_dim
        self.vocab, self.max_pos, self.eps, self.theta = vocab, max_pos, eps, theta
        self.tied, self.round_bf16 = tied, round_bf16

    def c(self) -> XoConfig:
        return XoConfig(self.hidden, self.inter, self.layers, self.q_heads, self.kv_heads,
                        self.head_dim, self.vocab, self.max_pos, self.eps, int(self.tied),
                        int(self.round_bf16))

    def tensors(self):
        cc = self.c()
        n = lib().xo_tensor_count(C.byref(cc))
        out = []
        buf = C.create_string_buffer(128)
        for i in range(n):
            size = lib().xo_tensor_info(C.byref(cc), i, buf, 128)
            out.append((buf.value.decode(), size))
        return out

    def to_json(self) -> dict:
        return {
            "model_type": "qwen3", "dtype": "bfloat16", "hidden_act": "silu",
            "attention_bias": False, "hidden_size": self.hidden,
            "intermediate_size": self.inter, "num_hidden_layers": self.layers,
            "num_attention_heads": self.q_heads, "num_key_value_heads": self.kv_heads,
            "head_dim": self.head_dim, "vocab_size": self.vocab,
            "max_position_embeddings": self.max_pos, "rms_norm_eps": self.eps,
            "rope_theta": self.theta, "tie_word_embeddings": bool(self.tied),
        }


class Model:
    """The reference forward (model.rs:155-279) over this library's weights."""

    def __init__(self, cfg: Config, weights_bf16: bool = True, inv_freq=None):
        self.cfg = cfg
        self._c = cfg.c()
        inv = inv_freq if inv_freq is not None else inv_freq_f32(cfg.head_dim, cfg.theta)
        self.inv_freq = f32(inv)
        self.bf16 = weights_bf16
        self.h = lib().xo_model_new(C.byref(self._c), self.inv_freq, int(weights_bf16))
        if not self.h:
            raise ValueError("oracle: config refused")
        self.names = [n for n, _ in cfg.tensors()]
        self.sizes = [s for _, s in cfg.tensors()]

    def __del__(self):
        if getattr(self, "h", None):
            lib().xo_model_free(self.h)
            self.h = None

    def set(self, name: str, values: np.ndarray):
        i = self.names.index(name)
        if self.bf16:
            a = np.ascontiguousarray(values).ravel()
            if a.dtype != np.uint16:
                a = bf16_bits(a)
        else:
            a = f32(values).ravel()
        assert a.size == self.sizes[i], (name, a.size, self.sizes[i])
        if lib().xo_model_set(self.h, i, 0, a.ctypes.data, a.size):
            raise ValueError(name)

    def init_normal(self, seed: int, std: float = 0.02):
        if lib().xo_model_init_normal(self.h, seed, std):
            raise ValueError("init_normal needs bf16 weights")

    def init_reference(self, seed: int):
        lib().xo_model_init_reference(self.h, seed)

    def reset(self):
        lib().xo_model_reset(self.h)

    def __len__(self):
        return lib().xo_model_len(self.h)

    def truncate(self, n: int):
        lib().xo_model_truncate(self.h, n)

    def step(self, token: int) -> np.ndarray:
        out = np.empty(self.cfg.vocab, np.float32)
        if lib().xo_model_step(self.h, token & 0xFFFFFFFF, out):
            raise ValueError("position past the model's")
        return out

    def extend(self, ids) -> np.ndarray:
        last = None
        for t in ids:
            last = self.step(int(t))
        return last

    def logits(self, ids):
        self.reset()
        return [self.step(int(t)) for t in ids]

    def cache_row(self, layer: int, pos: int):
        kvd = self.cfg.kv_heads * self.cfg.head_dim
        k, v = np.empty(kvd, np.float32), np.empty(kvd, np.float32)
        if lib().xo_model_cache_row(self.h, layer, pos, k, v):
            raise IndexError((layer, pos))
        return k, v

    def greedy(self, prompt, n: int):
        """Resets, feeds prompt, then n greedy tokens. Returns (tokens, top-2 margins)."""
        self.reset()
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.empty(n, np.uint32)
        margins = np.empty(n, np.float32)
        got = lib().xo_model_greedy(self.h, p, p.size, n, out, margins)
        return out[:got].copy(), margins[:got].copy()
