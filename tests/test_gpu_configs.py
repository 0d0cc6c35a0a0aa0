"""BASELINE.json configs 4 and 5 on the GPU.

Against the CPU oracle, at the layer widths of those configs (two layers, a 4096-token
vocabulary; tests/golden/make_oracle_long.py): config 4's 8192-token prompt through 2048-row
prefill passes, logits at and around every pass boundary and 16 greedy steps after it; config
5's 512-token prompt at Qwen3-32B widths. The f32 path within the model tolerance (0.05 of each
row's largest magnitude, KL <= 0.02, gpu_engine.rs:29-32); the exact mode (f64 sums) the oracle's
tokens and its logits to 1e-5 of the row scale.

At full size, where no oracle run fits: the Qwen3-8B prefill route (passes of 2048 rows) against
the decode route (one step per position) at the pass boundaries of an 8192-token prompt; batch 8
of 8192-token prompts and, at Qwen3-32B size, batch 16 of 512-token prompts, each sequence's
tokens and last logits the bits it gets alone."""
import json
import os

import numpy as np
import pytest

from common import LOGITS_ATOL_OF_MAX, LOGITS_KL, O

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def fixture(name):
    with open(os.path.join(HERE, "golden", f"oracle_long_{name}.json")) as fh:
        fx = json.load(fh)
    fx["rows_data"] = np.load(os.path.join(HERE, "golden", fx["rows"]), allow_pickle=False)
    fx["prompt"] = O.synthetic_ids(fx["prompt_len"], fx["config"]["vocab_size"], fx["prompt_seed"])
    return fx


def check_rows(what, got_rows, fx, exact):
    worst = 0.0
    for row, want, p in zip(got_rows, fx["rows_data"], fx["keep"]):
        scale = float(np.abs(want).max())
        err = float(np.abs(row.astype(np.float64) - want).max())
        if exact:
            assert err <= 1e-5 * scale, f"{what} position {p}: {err:.3e} from the oracle (scale {scale:.3f})"
        else:
            assert err <= LOGITS_ATOL_OF_MAX * scale, f"{what} position {p}: {err:.3e} (scale {scale:.3f})"
            assert O.kl(want, row) <= LOGITS_KL, f"{what} position {p}: KL"
            order = np.argsort(-want.astype(np.float64))
            if float(want[order[0]] - want[order[1]]) > 2 * LOGITS_ATOL_OF_MAX * scale:
                assert O.argmax(row) == int(order[0]), f"{what} position {p}: argmax"
        worst = max(worst, err / (LOGITS_ATOL_OF_MAX * scale))
    return worst


def check_greedy(what, tokens, fx, exact):
    g = fx["greedy"]
    want = np.array(g["tokens"], np.uint32)
    agree = next((i for i in range(want.size) if tokens[i] != want[i]), want.size)
    if exact:
        assert agree == want.size, f"{what}: greedy token {agree} differs from the oracle's"
    elif agree < want.size:
        tol = LOGITS_ATOL_OF_MAX * g["scales"][agree]
        assert g["margins"][agree] < 2 * tol, f"{what}: token {agree} differs at margin {g['margins'][agree]:.3e}"
    return agree


@pytest.mark.parametrize("name", ["8b", "32b"])
@pytest.mark.parametrize("f64", [False, True], ids=["f32", "f64"])
def test_two_layers_at_the_configs_widths_are_the_oracle(name, f64):
    from x0ne_core import Engine, EngineOptions, Route
    fx = fixture(name)
    prompt = fx["prompt"]
    e = Engine.load_synthetic(fx["config"], fx["seed"], fx["std"],
                              EngineOptions(max_ctx=prompt.size + 32, page_seed=11, f64_sums=f64))
    if not f64:
        assert f"prefill passes of {min(2048, prompt.size + 32)} rows" in e.describe(), e.describe()
    rows = e.logits_at(prompt, fx["keep"], Route.PREFILL)
    what = f"{fx['what']}, {'f64' if f64 else 'f32'} sums"
    worst = check_rows(what, rows, fx, f64)
    tokens = e.greedy(prompt, len(fx["greedy"]["tokens"]))
    agree = check_greedy(what, tokens, fx, f64)
    print(f"MEASURE {what}: kept logits within {worst:.4f} of the model tolerance; {agree} of "
          f"{len(tokens)} greedy tokens equal to the oracle's; {e.describe()}")
    assert e.client_data_is_zero()


QWEN3_8B = {"model_type": "qwen3", "dtype": "bfloat16", "hidden_act": "silu", "attention_bias": False,
            "hidden_size": 4096, "intermediate_size": 12288, "num_hidden_layers": 36, "num_attention_heads": 32,
            "num_key_value_heads": 8, "head_dim": 128, "vocab_size": 151936, "max_position_embeddings": 40960,
            "rms_norm_eps": 1e-6, "rope_theta": 1e6, "tie_word_embeddings": False}
QWEN3_32B = dict(QWEN3_8B, hidden_size=5120, intermediate_size=25600, num_hidden_layers=64, num_attention_heads=64)


def test_config4_prefill_passes_are_the_decode_route_at_full_size():
    """Qwen3-8B, an 8192-token prompt: the prefill route's logits (passes of 2048 rows through the
    matrix-core GEMMs and the causal attention) at and around every pass boundary against the
    decode route's (8192 decode steps), within the model tolerance."""
    from x0ne_core import Engine, EngineOptions, Route
    prompt = O.synthetic_ids(8192, QWEN3_8B["vocab_size"], 0)
    e = Engine.load_synthetic(QWEN3_8B, 0, 0.02, EngineOptions(max_ctx=8192 + 16, page_seed=1, f64_sums=False))
    assert "prefill passes of 2048 rows" in e.describe()
    keep = [2047, 2048, 4095, 4096, 6144, 8191]
    pre = e.logits_at(prompt, keep, Route.PREFILL)
    dec = e.logits_at(prompt, keep, Route.DECODE)
    worst = 0.0
    for a, b, p in zip(pre, dec, keep):
        scale = float(np.abs(b).max())
        err = float(np.abs(a.astype(np.float64) - b).max())
        worst = max(worst, err / (LOGITS_ATOL_OF_MAX * scale))
        assert err <= LOGITS_ATOL_OF_MAX * scale and O.kl(b, a) <= LOGITS_KL, f"position {p}: {err:.3e}"
    print(f"MEASURE Qwen3-8B 8192-token prompt: prefill route within {worst:.4f} of the tolerance of the decode route")
    assert e.client_data_is_zero()


@pytest.mark.parametrize("cfg,prompt_len,batch", [(QWEN3_8B, 8192, 8), (QWEN3_32B, 512, 16)],
                         ids=["config4-b8", "config5-b16"])
def test_a_full_size_batch_is_each_sequence_alone(cfg, prompt_len, batch):
    """Configs 4 (Qwen3-8B, 8 independent 8192-token prompts) and 5 (Qwen3-32B, 16 independent
    512-token prompts): the batched step's tokens and last logits for every sequence are the bits
    that sequence gets decoded alone on the same engine."""
    from x0ne_core import Engine, EngineOptions
    n = 8
    prompts = np.stack([O.synthetic_ids(prompt_len, cfg["vocab_size"], b) for b in range(batch)])
    e = Engine.load_synthetic(cfg, 0, 0.02, EngineOptions(max_ctx=prompt_len + n + 8, page_seed=3, max_batch=batch))
    toks, _, last = e.greedy_batch(prompts, n, logits=True)
    for b in range(batch):
        t1, _, l1 = e.greedy_batch(prompts[b:b + 1], n, logits=True)
        assert (t1[0] == toks[b]).all(), f"sequence {b}: tokens alone {t1[0].tolist()} in the batch {toks[b].tolist()}"
        assert (l1[0].view(np.uint32) == last[b].view(np.uint32)).all(), f"sequence {b}: last logits"
    print(f"MEASURE batch {batch} of {prompt_len}-token prompts: every sequence the bits it gets alone; "
          f"{e.describe()}")
    assert e.client_data_is_zero() and e.host_buffers_are_zero()
