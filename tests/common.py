"""Shared by the tests: deterministic data, checkpoints built in memory, comparisons — the
counterpart of x0ne-core/oracle/tests/common/mod.rs. The CPU oracle (oracle/) is the checker."""
from __future__ import annotations

import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "x0ne-engine_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

from oracle import oracle as O  # noqa: E402  (the checker)

# Tolerances (common/mod.rs:98-107).
BF16_RTOL = 1.0 / 128.0  # one bf16 ulp, relative
BF16_ATOL = 1e-6
F32_RTOL = 1e-5  # an f32 accumulation against an f64 one, share of sum |terms|
ATTENTION_ATOL_OF_VMAX = 1.0 / 128.0
ROPE_ATOL_OF_XMAX = 1e-3
# Model level (gpu_engine.rs:29-32).
LOGITS_ATOL_OF_MAX = 0.05
LOGITS_KL = 0.02


def bits_f32(v) -> np.ndarray:
    return np.ascontiguousarray(v, np.float32).view(np.uint32)


def bf16_bits(v) -> np.ndarray:
    return O.bf16_bits(np.asarray(v, np.float32))


def bf16_vals(b) -> np.ndarray:
    return O.bf16_values(np.asarray(b, np.uint16))


def max_abs(v) -> float:
    v = np.asarray(v, np.float64)
    v = v[np.isfinite(v)]
    return float(np.abs(v).max()) if v.size else 0.0


def worst_ratio(got, want, atol, rtol):
    """common/mod.rs:68-84: largest |got - want| / (atol + rtol |want|); two NaN or two equal
    values agree; a value not finite on one side only is infinitely far."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    assert got.shape == want.shape, (got.shape, want.shape)
    same = (np.isnan(got) & np.isnan(want)) | (got == want)
    fin = np.isfinite(got) & np.isfinite(want)
    with np.errstate(invalid="ignore", divide="ignore"):
        r = np.where(fin, np.abs(got - want) / (atol + rtol * np.abs(want)), np.inf)
    r = np.where(same, 0.0, r)
    if r.size == 0:
        return 0.0, 0
    i = int(np.argmax(r))
    return float(r[i]), i


def assert_close(what, got, want, atol, rtol):
    r, i = worst_ratio(got, want, atol, rtol)
    print(f"MEASURE {what}: worst ratio {r:.4f} (atol {atol:.3g}, rtol {rtol:.3g})")
    assert r <= 1.0, f"{what}: index {i}: got {np.asarray(got).ravel()[i]} want {np.asarray(want).ravel()[i]} (ratio {r:.3f})"


def bf16s_with_edges(rng: O.Rng, n: int, scale: float) -> np.ndarray:
    """gpu_kernels.rs:37-57: bf16 values with zeros of both signs, denormals and the extremes
    (one value in 16 on average)."""
    edges = np.array([0.0, -0.0, O.bf16_values(1)[0], O.bf16_values(0x8001)[0], O.bf16_values(0x007F)[0],
                      O.bf16_round(np.float32(scale))[0], O.bf16_round(np.float32(-scale))[0]], np.float32)
    out = rng.bf16s(n, scale)
    g = np.random.default_rng(rng.next_u64())
    mask = g.integers(0, 16, n) == 0
    out[mask] = edges[g.integers(0, len(edges), int(mask.sum()))]
    return out


def tiny(layers, q_heads, kv_heads, tied, **kw) -> O.Config:
    """common/mod.rs:181-195: a small model the kernels accept (head_dim 128, hidden % 8 == 0)."""
    c = dict(hidden=64, inter=96, layers=layers, q_heads=q_heads, kv_heads=kv_heads, head_dim=128, vocab=384,
             max_pos=2048, eps=1e-6, theta=1e6, tied=tied)
    c.update(kw)
    return O.Config(**c)


def wide() -> O.Config:
    """gpu_engine.rs:71-80"""
    return tiny(3, 16, 8, True, hidden=128, inter=256)


def oracle_model(cfg: O.Config, seed: int, init="reference") -> O.Model:
    m = O.Model(cfg, weights_bf16=True)
    if init == "reference":
        m.init_reference(seed)
    else:
        m.init_normal(seed, init)
    return m


def reference_tensors(cfg: O.Config, seed: int) -> dict:
    """common/mod.rs:199-221 restated over the splitmix64 stream: name -> (shape, bf16 bits)."""
    rng = O.Rng(seed)
    out = {}
    h, i, hd = cfg.hidden, cfg.inter, cfg.head_dim
    qd, kvd = cfg.q_heads * hd, cfg.kv_heads * hd
    for name, size in cfg.tensors():
        shape = tensor_shape(cfg, name)
        if len(shape) == 1:
            vals = np.array([O.bf16_round(np.float32(1.0) + np.float32(0.25) * np.float32(rng.unit()))[0]
                             for _ in range(size)], np.float32)
        elif "embed_tokens" in name or "lm_head" in name:
            vals = rng.bf16s(size, 1.0)
        else:
            vals = rng.bf16s(size, float(np.float32(2.0) / np.sqrt(np.float32(shape[1]))))
        out[name] = (shape, bf16_bits(vals))
    return out


def tensor_shape(cfg: O.Config, name: str):
    h, i, hd = cfg.hidden, cfg.inter, cfg.head_dim
    qd, kvd = cfg.q_heads * hd, cfg.kv_heads * hd
    if name in ("model.embed_tokens.weight", "lm_head.weight"):
        return [cfg.vocab, h]
    if name == "model.norm.weight":
        return [h]
    leaf = name.split(".", 3)[3].rsplit(".weight", 1)[0]
    return {"input_layernorm": [h], "post_attention_layernorm": [h], "self_attn.q_proj": [qd, h],
            "self_attn.k_proj": [kvd, h], "self_attn.v_proj": [kvd, h], "self_attn.q_norm": [hd],
            "self_attn.k_norm": [hd], "self_attn.o_proj": [h, qd], "mlp.gate_proj": [i, h],
            "mlp.up_proj": [i, h], "mlp.down_proj": [h, i]}[leaf]


def safetensors_bytes(tensors: dict, dtype="BF16") -> bytes:
    """A safetensors file of {name: (shape, uint16 bits)} laid out in order (common/mod.rs:120-153)."""
    header, at, blobs = {}, 0, []
    for name, (shape, bits) in tensors.items():
        b = np.ascontiguousarray(bits).tobytes()
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [at, at + len(b)]}
        at += len(b)
        blobs.append(b)
    h = json.dumps(header).encode()
    return len(h).to_bytes(8, "little") + h + b"".join(blobs)


def oracle_from_tensors(cfg: O.Config, tensors: dict) -> O.Model:
    m = O.Model(cfg, weights_bf16=True)
    for name, (_, bits) in tensors.items():
        if name in m.names:
            m.set(name, bits)
    return m


def top_two(row):
    s = np.sort(np.asarray(row, np.float32))
    return float(s[-1]), float(s[-2])
