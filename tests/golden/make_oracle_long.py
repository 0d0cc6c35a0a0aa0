"""Writes tests/golden/oracle_long_<name>.json and .npy: the CPU oracle on a two-layer model at the
widths of BASELINE.json's long-context and 32B configurations, with N(0, 0.02) bf16 weights drawn
from seed 0 (norm weights 1.0, the device initialiser's draws) and a 4096-token vocabulary (the
LM head is not a layer width; a full vocabulary would multiply the oracle's time by forty):

- 8b: hidden 4096, intermediate 12288, 32 q / 8 kv heads; an 8192-token splitmix64 prompt, the
  length config 4 prefills in 2048-row passes, logits kept around every pass boundary.
- 32b: hidden 5120, intermediate 25600, 64 q / 8 kv heads; config 5's 512-token prompt.

Each keeps the f32 logits rows at the kept positions (.npy, [keep][vocab]) and 16 greedy steps
after the prompt (token, top-2 margin, row scale, log-sum-exp, top-16 ids and logits).

usage: make_oracle_long.py 8b|32b
"""
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from oracle import oracle as O  # noqa: E402

VOCAB = 4096
SHAPES = {
    "8b": dict(hidden=4096, inter=12288, q_heads=32, kv_heads=8, prompt=8192,
               keep=[0, 2046, 2047, 2048, 2049, 4095, 4096, 6143, 6144, 8190, 8191]),
    "32b": dict(hidden=5120, inter=25600, q_heads=64, kv_heads=8, prompt=512, keep=[0, 255, 256, 510, 511]),
}
STEPS, TOP = 16, 16


def main():
    name = sys.argv[1]
    s = SHAPES[name]
    cfg = O.Config(s["hidden"], s["inter"], 2, s["q_heads"], s["kv_heads"], 128, VOCAB, 40960, eps=1e-6, theta=1e6,
                   tied=False)
    O.set_threads(os.cpu_count() or 8)
    m = O.Model(cfg, weights_bf16=True)
    t = time.time()
    m.init_normal(0, 0.02)
    prompt = O.synthetic_ids(s["prompt"], VOCAB, 0)
    m.reset()
    rows = []
    row = None
    for p, tok in enumerate(prompt):
        row = m.step(int(tok))
        if p in s["keep"]:
            rows.append(row.copy())
        if p % 512 == 0:
            print(f"{name}: position {p} at {time.time() - t:.0f} s", flush=True)
    steps = {"tokens": [], "margins": [], "scales": [], "logsumexp": [], "top_ids": [], "top_logits": []}
    for i in range(STEPS):
        order = np.argsort(-row.astype(np.float64), kind="stable")[:TOP]
        tok = O.argmax(row)
        steps["tokens"].append(tok)
        steps["margins"].append(float(row[order[0]]) - float(row[order[1]]))
        steps["scales"].append(float(np.abs(row).max()))
        steps["logsumexp"].append(O.logsumexp(row))
        steps["top_ids"].append([int(x) for x in order])
        steps["top_logits"].append([float(row[x]) for x in order])
        if i + 1 < STEPS:
            row = m.step(tok)
    base = os.path.join(HERE, f"oracle_long_{name}")
    np.save(base + ".npy", np.stack(rows).astype(np.float32))
    out = {"what": f"CPU oracle, two layers at Qwen3-{name} widths, vocabulary {VOCAB}, N(0,0.02) bf16 weights "
                   f"from seed 0 (norms 1.0), a {s['prompt']}-token splitmix64 seed-0 prompt",
           "config": cfg.to_json(), "seed": 0, "std": 0.02, "prompt_len": s["prompt"], "prompt_seed": 0,
           "keep": s["keep"], "rows": os.path.basename(base + ".npy"), "greedy": steps,
           "seconds": round(time.time() - t, 1)}
    with open(base + ".json", "w") as fh:
        json.dump(out, fh, indent=0)
    print(name, steps["tokens"], round(time.time() - t, 1), "s")


if __name__ == "__main__":
    main()
