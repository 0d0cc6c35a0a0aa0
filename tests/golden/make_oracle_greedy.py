"""Writes tests/golden/oracle_greedy_<name>.json: the CPU oracle's greedy continuation of the
bench workload (N(0, 0.02) bf16 weights drawn from seed 0, a 20-token splitmix64 seed-0 prompt).
Per step it keeps the chosen token, the top-1 minus top-2 logit margin, the row's largest logit
magnitude (the scale of the model-level tolerance), its log-sum-exp, and the 16 largest logits
with their ids: enough for a GPU test to check the engine's logits at every generated position,
not only its argmax. The oracle (oracle/) restates the reference's Rust oracle.

usage: make_oracle_greedy.py 8b|0.6b [steps]
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

SHAPES = {
    "8b": dict(hidden=4096, inter=12288, layers=36, q_heads=32, kv_heads=8, tied=False),
    "0.6b": dict(hidden=1024, inter=3072, layers=28, q_heads=16, kv_heads=8, tied=True),
    "32b": dict(hidden=5120, inter=25600, layers=64, q_heads=64, kv_heads=8, tied=False),
}
TOP = 16


def main():
    name = sys.argv[1]
    steps = int(sys.argv[2]) if len(sys.argv) > 2 else 64
    s = SHAPES[name]
    cfg = O.Config(s["hidden"], s["inter"], s["layers"], s["q_heads"], s["kv_heads"], 128, 151936, 40960,
                   eps=1e-6, theta=1e6, tied=s["tied"])
    O.set_threads(os.cpu_count() or 8)
    m = O.Model(cfg, weights_bf16=True)
    t = time.time()
    m.init_normal(0, 0.02)
    prompt = O.synthetic_ids(20, 151936, 0)
    m.reset()
    row = m.extend(prompt)
    toks, margins, scales, lses, top_ids, top_vals = [], [], [], [], [], []
    for i in range(steps):
        order = np.argsort(-row.astype(np.float64), kind="stable")[:TOP]
        tok = O.argmax(row)
        assert tok == int(order[0])
        toks.append(tok)
        margins.append(float(row[order[0]]) - float(row[order[1]]))
        scales.append(float(np.abs(row).max()))
        lses.append(O.logsumexp(row))
        top_ids.append([int(x) for x in order])
        top_vals.append([float(row[x]) for x in order])
        if i + 1 < steps:
            row = m.step(tok)
    out = {"what": f"CPU-oracle greedy, Qwen3-{name} shape, N(0,0.02) bf16 weights from seed 0 (norms 1.0)",
           "config": cfg.to_json(), "seed": 0, "std": 0.02, "prompt": prompt.tolist(), "tokens": toks,
           "margins": margins, "scales": scales, "logsumexp": lses, "top_ids": top_ids, "top_logits": top_vals,
           "seconds": round(time.time() - t, 1)}
    with open(os.path.join(HERE, f"oracle_greedy_{name.replace('.', '_')}.json"), "w") as fh:
        json.dump(out, fh, indent=0)
    print(out["tokens"][:16], min(out["margins"]), out["seconds"])


if __name__ == "__main__":
    main()
