"""Copies the reference's data fixtures for this path into tests/golden/ (run once, in the
container that holds /root/reference; the copies are committed, the reference never travels).

- x0ne-infer/tests/arch/qwen3/{config.json, model.safetensors, reference.json}: a tiny Qwen3
  (head_dim 8, 3 q heads / 1 kv head, 4 layers, vocab 40, theta 1e4, tied, F32) with the logits
  transformers 5.17 computed for 12 ids and its greedy continuation of a 6-id prompt
  (made by x0ne-infer/scripts/make-arch-fixtures.py; checked by the reference at 1e-4 in
  x0ne-infer/src/decoder.rs:460-471 and greedy-equal in qwen3.rs:790-821).
- the known-answer synthetic ids of x0ne-infer/src/bench_tests.rs:1072-1081 (seed 0x0C0E5EED,
  vocab 151936), written as JSON data.
"""
import hashlib
import json
import os
import shutil

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))


def main():
    src = os.path.join(REF, "x0ne-infer/tests/arch/qwen3")
    dst = os.path.join(HERE, "arch_qwen3")
    os.makedirs(dst, exist_ok=True)
    sums = {}
    for f in ("config.json", "model.safetensors", "reference.json"):
        shutil.copyfile(os.path.join(src, f), os.path.join(dst, f))
        with open(os.path.join(dst, f), "rb") as fh:
            sums[f] = hashlib.sha256(fh.read()).hexdigest()
    with open(os.path.join(dst, "SHA256SUMS.json"), "w") as fh:
        json.dump({"source": "x0ne-infer/tests/arch/qwen3", "sha256": sums}, fh, indent=1)
    kat = {
        "source": "x0ne-infer/src/bench_tests.rs:1072-1081 (the_synthetic_ids_are_core_bench_s)",
        "generator": "splitmix64, below(n) = next_u64 % n (x0ne-core/oracle/examples/core-perf.rs:17-28)",
        "seed": 0x0C0E5EED,
        "vocab": 151936,
        "ids": [126819, 135692, 59481, 30850, 145817, 72711],
        "bound_check": {"n": 40000, "vocab": 1000},
    }
    with open(os.path.join(HERE, "synthetic_ids.json"), "w") as fh:
        json.dump(kat, fh, indent=1)


if __name__ == "__main__":
    main()
