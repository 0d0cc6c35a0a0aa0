"""The CPU oracle pinned to the reference's own fixtures (no GPU):

- the known-answer synthetic ids (x0ne-infer/src/bench_tests.rs:1072-1081);
- the transformers 5.17 Qwen3 fixture x0ne-infer/tests/arch/qwen3: logits within 1e-4 (the
  reference's own check of its decoder, x0ne-infer/src/decoder.rs:460-471) and the greedy
  continuation exactly (qwen3.rs:790-821). It fixes the model's mathematics: norm placement,
  per-head QK-norm, rotate-half RoPE, GQA head mapping, SwiGLU, tied embeddings.
"""
import json
import os

import numpy as np
import pytest

from common import O, ROOT

GOLDEN = os.path.join(ROOT, "tests", "golden")


def test_synthetic_ids_are_the_references_known_answer():
    kat = json.load(open(os.path.join(GOLDEN, "synthetic_ids.json")))
    ids = O.synthetic_ids(len(kat["ids"]), kat["vocab"], kat["seed"])
    assert ids.tolist() == kat["ids"]
    b = kat["bound_check"]
    assert (O.synthetic_ids(b["n"], b["vocab"], kat["seed"]) < b["vocab"]).all()


def arch_model():
    from safetensors.numpy import load_file
    d = os.path.join(GOLDEN, "arch_qwen3")
    cfg = json.load(open(os.path.join(d, "config.json")))
    ref = json.load(open(os.path.join(d, "reference.json")))
    w = load_file(os.path.join(d, "model.safetensors"))
    c = O.Config(cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"],
                 cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"], cfg["vocab_size"],
                 cfg["max_position_embeddings"], eps=cfg["rms_norm_eps"],
                 theta=cfg["rope_parameters"]["rope_theta"], tied=cfg["tie_word_embeddings"], round_bf16=False)
    m = O.Model(c, weights_bf16=False)
    assert sorted(m.names) == sorted(w), "the fixture holds exactly the checkpoint's tensors"
    for name in m.names:
        m.set(name, w[name])
    return m, ref


def test_the_forward_is_transformers_on_the_reference_fixture():
    m, ref = arch_model()
    got = np.array(m.logits(ref["ids"]))
    want = np.array(ref["logits"], np.float32).reshape(len(ref["ids"]), -1)
    err = float(np.abs(got - want).max())
    print(f"MEASURE transformers fixture: max |logit - reference| {err:.3e} (scale {np.abs(want).max():.2f})")
    assert err <= 1e-4


def test_greedy_is_transformers_on_the_reference_fixture():
    m, ref = arch_model()
    toks, margins = m.greedy(ref["prompt"], len(ref["generated"]))
    assert toks.tolist() == ref["generated"]


def test_a_plausible_mistake_fails_the_fixture():
    """The fixture catches the mistakes it is there for: the rotation's sign, the GQA mapping."""
    m, ref = arch_model()
    want = np.array(ref["logits"], np.float32).reshape(len(ref["ids"]), -1)
    # A transposed o_proj (a wrong operand) moves the logits well past the tolerance.
    from safetensors.numpy import load_file
    w = load_file(os.path.join(GOLDEN, "arch_qwen3", "model.safetensors"))
    name = "model.layers.1.self_attn.o_proj.weight"
    wo = w[name]
    m.set(name, wo[:, ::-1].copy())
    got = np.array(m.logits(ref["ids"]))
    assert np.abs(got - want).max() > 1e-2
    # The wrong RoPE theta (1e6 instead of the fixture's 1e4) does too, from position 1 on.
    m.set(name, wo)
    cfg = m.cfg
    bad = O.Config(cfg.hidden, cfg.inter, cfg.layers, cfg.q_heads, cfg.kv_heads, cfg.head_dim, cfg.vocab,
                   cfg.max_pos, eps=cfg.eps, theta=1e6, tied=True, round_bf16=False)
    mb = O.Model(bad, weights_bf16=False)
    for n in mb.names:
        mb.set(n, w[n])
    got = np.array(mb.logits(ref["ids"]))
    assert np.abs(got[0] - want[0]).max() <= 1e-4, "position 0 does not rotate"
    assert np.abs(got[1:] - want[1:]).max() > 1e-3
