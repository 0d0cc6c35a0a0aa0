"""An independent pin of the oracle's bf16 decode step (oracle/x0ne_oracle.c xo_model_step, which
restates x0ne-core/oracle/src/model.rs:196-262): the same step written again here in numpy
float64, each of its eleven bf16 rounding points explicit, compared with the C oracle bit for
bit on small models (GQA 1/1, 4/2 and 16/8, untied and tied). A mutation check then drops each
rounding point in turn from the numpy step: every one of them must change the logits' bits, so
a C oracle that missed or misplaced one would fail this test.

Nothing here calls the C oracle's kernels: the numpy step has its own embedding, add + RMSNorm,
GEMV, QK-norm + RoPE, attention, SwiGLU and bf16 rounding (RNE on the f32 bits, a NaN keeping its
sign with the quiet bit, oracle/src/bf16.rs:5-54). Sine, cosine and exp come from Python's math
module (the platform libm the C oracle calls too); sums are numpy float64 dot products, whose
order differs from the oracle's loops by about 1e-16 relative, far below the f32 and bf16
roundings the outputs are compared at."""
import math

import numpy as np
import pytest

from common import O, reference_tensors, tiny, wide

POINTS = ["input_norm", "qkv", "k_cache", "q", "attention", "o_proj", "post_norm", "gate_up", "swiglu",
          "down", "final_norm"]


def bf16(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 -> f32, round to nearest even on the bits; NaN keeps its sign, gets the quiet
    bit (bf16.rs:11-20)."""
    b = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    nan = np.isnan(np.asarray(x, np.float32))
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((b >> 16) | 0x40) & 0xFFFF, r)
    return (r.astype(np.uint32) << 16).view(np.float32)


class NumpyStep:
    """model.rs:196-262 in numpy float64, over the checkpoint's f32 values (bf16 numbers)."""

    def __init__(self, cfg, tensors, inv_freq, skip=()):
        self.c = cfg
        self.w = {k: O.bf16_values(bits).astype(np.float32).reshape(shape) for k, (shape, bits) in tensors.items()}
        self.inv = np.asarray(inv_freq, np.float32)
        self.skip = set(skip)
        self.k = [[] for _ in range(cfg.layers)]
        self.v = [[] for _ in range(cfg.layers)]

    def r(self, point, x):
        return x if point in self.skip else bf16(x)

    def add_rmsnorm(self, residual, x, w):
        residual += np.asarray(x, np.float32)  # one f32 addition per value
        r64 = residual.astype(np.float64)
        scale = 1.0 / math.sqrt(float(np.dot(r64, r64)) / r64.size + float(np.float32(self.c.eps)))
        return (r64 * scale * w.astype(np.float64)).astype(np.float32)

    @staticmethod
    def gemv(w, x):
        return (w.astype(np.float64) @ np.asarray(x, np.float64)).astype(np.float32)

    def norm_rope(self, x, w, pos):
        hd = self.c.head_dim
        half = hd // 2
        x64 = x.astype(np.float64)
        scale = 1.0 / math.sqrt(float(np.dot(x64, x64)) / hd + float(np.float32(self.c.eps)))
        n = x64 * scale * w.astype(np.float64)
        out = np.empty(hd, np.float32)
        for i in range(half):
            angle = float(np.float32(np.float32(pos) * self.inv[i]))
            s, c = math.sin(angle), math.cos(angle)
            out[i] = np.float32(n[i] * c - n[i + half] * s)
            out[i + half] = np.float32(n[i + half] * c + n[i] * s)
        return out

    def attend(self, q, K, V):
        scale = 1.0 / math.sqrt(self.c.head_dim)
        s = (K.astype(np.float64) @ q.astype(np.float64)) * scale
        m = s.max()
        p = np.array([math.exp(v - m) for v in s])
        out = (p @ V.astype(np.float64)) / p.sum()
        return out.astype(np.float32)

    def step(self, token, pos):
        c, W = self.c, self.w
        h, hd = c.hidden, c.head_dim
        qd, kvd = c.q_heads * hd, c.kv_heads * hd
        grp = c.q_heads // c.kv_heads
        emb = W["model.embed_tokens.weight"]
        delta = emb[token].copy() if token < c.vocab else np.zeros(h, np.float32)
        residual = np.zeros(h, np.float32)
        for l in range(c.layers):
            p = f"model.layers.{l}."
            x = self.r("input_norm", self.add_rmsnorm(residual, delta, W[p + "input_layernorm.weight"]))
            wqkv = np.concatenate([W[p + "self_attn.q_proj.weight"], W[p + "self_attn.k_proj.weight"],
                                   W[p + "self_attn.v_proj.weight"]])
            qkv = self.r("qkv", self.gemv(wqkv, x))
            q = np.concatenate([self.norm_rope(qkv[i * hd:(i + 1) * hd], W[p + "self_attn.q_norm.weight"], pos)
                                for i in range(c.q_heads)])
            k = np.concatenate([self.norm_rope(qkv[qd + i * hd:qd + (i + 1) * hd], W[p + "self_attn.k_norm.weight"],
                                               pos) for i in range(c.kv_heads)])
            self.k[l].append(self.r("k_cache", k))
            self.v[l].append(qkv[qd + kvd:].copy())
            q = self.r("q", q)
            K, V = np.stack(self.k[l]), np.stack(self.v[l])
            attn = np.concatenate([self.attend(q[hh * hd:(hh + 1) * hd], K[:, (hh // grp) * hd:(hh // grp + 1) * hd],
                                               V[:, (hh // grp) * hd:(hh // grp + 1) * hd])
                                   for hh in range(c.q_heads)])
            attn = self.r("attention", attn)
            delta = self.r("o_proj", self.gemv(W[p + "self_attn.o_proj.weight"], attn))
            x = self.r("post_norm", self.add_rmsnorm(residual, delta, W[p + "post_attention_layernorm.weight"]))
            gu = self.r("gate_up", self.gemv(np.concatenate([W[p + "mlp.gate_proj.weight"],
                                                              W[p + "mlp.up_proj.weight"]]), x))
            g, u = gu[:c.inter].astype(np.float64), gu[c.inter:].astype(np.float64)
            act = np.array([gi / (1.0 + math.exp(-gi)) * ui for gi, ui in zip(g, u)]).astype(np.float32)
            act = self.r("swiglu", act)
            delta = self.r("down", self.gemv(W[p + "mlp.down_proj.weight"], act))
        x = self.r("final_norm", self.add_rmsnorm(residual, delta, W["model.norm.weight"]))
        head = W["model.embed_tokens.weight"] if c.tied else W["lm_head.weight"]
        return self.gemv(head, x)


CONFIGS = [("1 layer 1/1", lambda: tiny(1, 1, 1, False)), ("2 layers 4/2", lambda: tiny(2, 4, 2, False)),
           ("2 layers 4/2 tied", lambda: tiny(2, 4, 2, True)), ("3 layers 16/8 tied", wide)]


def oracle_rows(cfg, tensors, inv, ids):
    m = O.Model(cfg, weights_bf16=True, inv_freq=inv)
    for name, (_, b) in tensors.items():
        m.set(name, b)
    return m.logits(ids)


def inv_freq_np(cfg):
    """ops.rs:210-214's f32 inverse frequencies, computed here once and given to both steps."""
    return np.array([np.float32(1.0) / np.float32(math.pow(cfg.theta, (2 * i) / cfg.head_dim))
                     for i in range(cfg.head_dim // 2)], np.float32)


@pytest.mark.parametrize("name,make", CONFIGS, ids=[c[0] for c in CONFIGS])
def test_the_oracle_step_is_the_numpy_restatement_bit_for_bit(name, make):
    cfg = make()
    tensors = reference_tensors(cfg, 70 + cfg.layers)
    inv = inv_freq_np(cfg)
    ids = O.Rng(71).tokens(12, cfg.vocab)
    ids[5] = cfg.vocab  # a token outside the vocabulary: a zero embedding row
    want = oracle_rows(cfg, tensors, inv, ids)
    ref = NumpyStep(cfg, tensors, inv)
    for pos, t in enumerate(ids):
        got = ref.step(int(t), pos)
        same = got.view(np.uint32) == want[pos].view(np.uint32)
        assert same.all(), f"{name} position {pos}: {int((~same).sum())} of {same.size} logits differ"


def test_every_rounding_point_of_the_step_changes_its_bits():
    """Dropped one at a time from the numpy step, each of the eleven bf16 rounding points moves
    the logits away from the oracle's bits: the comparison above would see an oracle without it."""
    cfg = tiny(2, 4, 2, False)
    tensors = reference_tensors(cfg, 72)
    inv = inv_freq_np(cfg)
    ids = O.Rng(73).tokens(10, cfg.vocab)
    want = oracle_rows(cfg, tensors, inv, ids)
    for point in POINTS:
        ref = NumpyStep(cfg, tensors, inv, skip=[point])
        differ = 0
        for pos, t in enumerate(ids):
            differ += int((ref.step(int(t), pos).view(np.uint32) != want[pos].view(np.uint32)).sum())
        print(f"MEASURE without the {point} rounding: {differ} of {len(ids) * cfg.vocab} logits differ")
        assert differ > 0, f"dropping the {point} rounding left every logit's bits unchanged"


def test_the_numpy_bf16_rounding_is_the_oracles():
    """The restatement's rounding against the oracle's encoder, on every upper half and the
    deciding lower halves (ties, just below and above, NaN payloads)."""
    hi = np.arange(1 << 16, dtype=np.uint32) << 16
    for lo in [0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF]:
        x = (hi | lo).view(np.float32)
        got = bf16(x).view(np.uint32) >> 16
        want = O.bf16_bits(x).astype(np.uint32)
        assert (got == want).all(), f"lower half {lo:#06x}"
