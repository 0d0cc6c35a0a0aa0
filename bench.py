#!/usr/bin/env python3
"""Qwen3-8B bf16 batch-1 greedy decode on one MI355X, the metric BASELINE.json names:
"Qwen3-8B bf16 decode tok/s @batch1; decode HBM GB/s vs 8 TB/s peak".

Workload: Qwen3-8B shape (36 layers, hidden 4096, 32 q / 8 kv heads,
head_dim 128, intermediate 12288, vocab 151936, untied), random-init bf16 weights N(0, 0.02) drawn
on the device from seed 0 (norm weights 1.0), a 20-token prompt of uniform random ids
(splitmix64 seed 0), then greedy decode steps at batch 1, each step one replay of the captured
HIP graph. A step is one decode step (one token); W untimed steps, then exactly K steps timed
between two stream synchronisations. value = K / seconds. The timed path is the engine's default,
the exact mode (f64 sums in the projections and attention, the oracle's rounding points, so the
greedy tokens are the oracle's); --f32-sums times the fp32-accumulating path instead, and the
other of the two is timed after it on the same workload (parity.other_mode).

Also printed, in the same JSON line:
- roofline: the dominant kernel (the gate/up GEMV with its fused RMSNorm and SwiGLU, 201 MB of
  weights per launch) timed alone with HIP events on the engine's stream over every layer's
  weights; achieved = algorithmic bytes per launch / average launch time, against 8 TB/s.
- decode_hbm: bytes per step (roofline.rs formula: every weight once + K/V of the attended
  positions) x steps / s, against 8 TB/s.
- cpu_baseline: the CPU oracle (oracle/, a C restatement of the reference's Rust oracle, f64
  inside) on this host's cores, on a bounded sample of the same workload.
- prefill: the prompt's time to the first token (greedy_timed's first host time: the prompt in
  passes of up to 2048 rows, the f32 path through bf16 matrix-core GEMMs and the causal prefill
  attention, the exact mode through the f64-sum GEMM on the f64 matrix cores and the f64 causal
  attention; then the LM head on the last row), as tok/s and TFLOP/s against the dense peak of
  the arithmetic it runs in (bf16 2.5 PFLOP/s; the exact mode's f64 78.6 TFLOP/s).

--prompt 8192 --steps 512 is BASELINE.json config 4 (8B, 8192-token prompt, 512 decode steps);
--model 32b --prompt 512 is config 5's batch-1 case; --model 0.6b --steps 64 config 1's.
--batch B decodes B independent prompts (splitmix64 seeds 0 .. B - 1; sequence 0's is the batch-1
prompt) together, each step one replay of the batched step's graph: config 4 at batch 8 is
--prompt 8192 --steps 512 --batch 8, config 5 at batch 16 --model 32b --prompt 512 --batch 16.
value is then B x K / seconds (tokens of all sequences), the roofline kernel the batched gate/up
projection (the few-row matrix-core GEMM with SwiGLU behind).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, os.path.join(ROOT, "x0ne-engine_amd")):
    if p not in sys.path:
        sys.path.insert(0, p)

QWEN3_8B = {
    "model_type": "qwen3", "dtype": "bfloat16", "hidden_act": "silu", "attention_bias": False,
    "hidden_size": 4096, "intermediate_size": 12288, "num_hidden_layers": 36, "num_attention_heads": 32,
    "num_key_value_heads": 8, "head_dim": 128, "vocab_size": 151936, "max_position_embeddings": 40960,
    "rms_norm_eps": 1e-6, "rope_theta": 1e6, "tie_word_embeddings": False,
}
QWEN3_32B = dict(QWEN3_8B, hidden_size=5120, intermediate_size=25600, num_hidden_layers=64,
                 num_attention_heads=64, num_key_value_heads=8)
QWEN3_0_6B = dict(QWEN3_8B, hidden_size=1024, intermediate_size=3072, num_hidden_layers=28, num_attention_heads=16,
                  num_key_value_heads=8, tie_word_embeddings=True)
MODELS = {"8b": ("Qwen3-8B", QWEN3_8B), "32b": ("Qwen3-32B", QWEN3_32B), "0.6b": ("Qwen3-0.6B", QWEN3_0_6B)}
PROMPT = 20
SEED = 0
STD = 0.02


def splitmix_ids(n: int, vocab: int, seed: int) -> np.ndarray:
    """Uniform ids from splitmix64 (oracle/tests/common/mod.rs:15-25; core-perf.rs:17-28)."""
    out, s = [], seed
    M = (1 << 64) - 1
    for _ in range(n):
        s = (s + 0x9E3779B97F4A7C15) & M
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        out.append((z ^ (z >> 31)) % vocab)
    return np.array(out, np.uint32)


def cpu_threads() -> int:
    """The host threads of the CPU leg: the GPU box's CPU share per GPU (its OMP_NUM_THREADS, 16
    on the box), else every core this host has."""
    return int(os.environ.get("OMP_NUM_THREADS", "0")) or (os.cpu_count() or 1)


def cpu_baseline(cfg: dict, prompt: np.ndarray, threads: int, steps: int = 8, prompt_len: int = 4,
                 name: str = "Qwen3-8B") -> dict:
    """The CPU oracle on the same shape and weights (drawn by the oracle's generator, the same
    bits as the device's): a `prompt_len`-token prompt, then `steps` greedy decode steps; tok/s
    over the decode steps. Also one thread on two steps, the reference oracle being
    single-threaded."""
    from oracle import oracle as O
    c = O.Config(cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"],
                 cfg["num_attention_heads"], cfg["num_key_value_heads"], cfg["head_dim"], cfg["vocab_size"],
                 cfg["max_position_embeddings"], eps=cfg["rms_norm_eps"], theta=cfg["rope_theta"],
                 tied=cfg["tie_word_embeddings"])
    O.set_threads(threads)
    m = O.Model(c, weights_bf16=True)
    t = time.perf_counter()
    m.init_normal(SEED, STD)
    init_s = time.perf_counter() - t
    m.reset()
    logits = m.extend(prompt[:prompt_len])
    times = []
    t0 = time.perf_counter()
    for _ in range(steps):
        tok = O.argmax(logits)
        logits = m.step(tok)
        times.append(time.perf_counter() - t0)
    value = steps / times[-1]
    O.set_threads(1)
    single_steps = 2
    t0 = time.perf_counter()
    for _ in range(single_steps):
        logits = m.step(O.argmax(logits))
    single = single_steps / (time.perf_counter() - t0)
    O.set_threads(threads)
    return {"value": round(value, 4), "unit": "tok/s", "cores": threads, "kind": "port",
            "single_thread_value": round(single, 4),
            "sample": f"{name} shape, the same N(0,{STD}) bf16 weights (seed {SEED}, drawn by the oracle's "
                      f"generator in {init_s:.1f} s, not timed), {prompt_len}-token prompt, {steps} greedy decode "
                      f"steps timed on {threads} threads (rows split, f64 sums in the reference's order; the "
                      f"GPU box's CPU share per GPU); single_thread_value: {single_steps} more steps on 1 thread, "
                      f"as the reference's oracle runs"}


TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "qwen3-8b-decode_hbm-bytes.md")


BATCH8_TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "qwen3-8b-decode-batch8_hbm-bytes.md")


ATTENTION_TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "decode-attention-8k-32k_hbm-bytes.md")


def measured_traffic(kernel: str, profile: str = TRAFFIC_PROFILE):
    """HBM bytes per launch of `kernel` from a committed rocprofv3 byte-counter summary
    (FETCH_SIZE and WRITE_SIZE runs, scaled by a copy of known size), or None."""
    import re
    try:
        with open(profile) as fh:
            m = re.search(rf"^traffic_bytes_per_launch {kernel} = (\d+)$", fh.read(), re.M)
    except OSError:
        return None
    return int(m.group(1)) if m else None


def copy_calibration(n: int):
    """One device-to-device hipMemcpy of n bytes (the runtime's plain copy kernel): a known
    number of bytes read and written, for scaling the hardware's byte counters."""
    import ctypes as C
    hip = C.CDLL("libamdhip64.so")
    src, dst = C.c_void_p(), C.c_void_p()
    for p in (src, dst):
        if hip.hipMalloc(C.byref(p), C.c_size_t(n)) != 0:
            raise SystemExit("calibration copy: hipMalloc failed")
    try:
        if hip.hipMemset(src, 1, C.c_size_t(n)) != 0 or hip.hipDeviceSynchronize() != 0:
            raise SystemExit("calibration copy: hipMemset failed")
        if hip.hipMemcpy(dst, src, C.c_size_t(n), 3) != 0 or hip.hipDeviceSynchronize() != 0:  # device to device
            raise SystemExit("calibration copy: hipMemcpy failed")
    finally:
        hip.hipFree(src)
        hip.hipFree(dst)
    print(f"[bench] calibration copy: {n} bytes read, {n} bytes written", file=sys.stderr, flush=True)


def attention_line(args) -> dict:
    """the isolated decode attention (Qwen3-8B geometry, 32 q / 8 kv heads)
    at ctx 1k / 8k / 32k and P in {1, 4, 16} (the configuration's) and 32 (the engine's), each
    launch over distinct K/V planes (more than
    512 MiB rotated); bytes per launch 2 ctx 8 128 2 (K + V) + Q + out + the split states. The
    table also holds P 64 and 128 (two and four rounds of blocks), which the value does not use."""
    from x0ne_core.gpu import Gpu
    g = Gpu()
    qh, kvh = 32, 8
    rows = []
    cases = [(c, p) for c in (1024, 8192, 32768) for p in (1, 4, 16, 32, 64, 128)]
    if args.attention_case:  # one (ctx, P), e.g. for a counter run whose dispatches are all that case
        c, p = (int(v) for v in args.attention_case.split(":"))
        cases = [(c, p)]
    if args.calibrate_copy:
        copy_calibration(args.calibrate_copy << 20)
    for ctx, P in cases:
        us, planes = g.time_attention(qh, kvh, ctx, P, args.attention_iters, SEED)
        nbytes = 2 * ctx * kvh * 128 * 2 + qh * 128 * 2 * 2 + (qh * P * 132 * 4 if P > 1 else 0)
        rows.append({"ctx": ctx, "splits": P, "us": round(us, 3), "gbs": round(nbytes / us / 1e3, 1),
                     "frac": round(nbytes / us / 1e3 / 8000.0, 4), "bytes": nbytes, "planes": planes})
        print(f"[bench] attention ctx {ctx} P {P}: {us:.2f} us, {nbytes / us / 1e3:.1f} GB/s ({planes} planes)",
              file=sys.stderr, flush=True)
    best = max((r for r in rows if r["ctx"] == max(c for c, _ in cases) and r["splits"] <= 32), key=lambda r: r["gbs"])
    return {
        "metric": "Qwen3-8B decode attention GB/s (BASELINE.json config 2) vs 8 TB/s peak",
        "value": best["gbs"], "unit": "GB/s", "n_gpus": 1, "steps": args.attention_iters, "warmup": 0,
        "ms_per_step": round(best["us"] / 1e3, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16", "data": "synthetic: Q, K, V N(0,1) bf16 (seed 0), pages in a seeded permutation",
        "config": {"workload": "isolated split-K decode attention, 32q/8kv heads, head_dim 128, last-block merge; "
                               "value at ctx 32768 with the fastest P", "ctx": best["ctx"], "splits": best["splits"],
                   "table": rows},
        "roofline": {"kernel": "x0ne_attention_decode_split_g4_bf16", "bound": "hbm", "achieved": best["gbs"],
                     "peak": 8000.0, "unit": "GB/s", "frac": best["frac"],
                     "traffic": measured_traffic(f"attention_{best['ctx']}_{best['splits']}", ATTENTION_TRAFFIC_PROFILE),
                     "traffic_source": os.path.relpath(ATTENTION_TRAFFIC_PROFILE, ROOT),
                     "bytes_per_launch": best["bytes"], "avg_us": best["us"],
                     "timing": "hipExtLaunchKernel start/stop events per launch"},
    }


def batch_line(args, model_name: str, cfg: dict) -> dict:
    """--batch B: B independent prompts decoded together (the batched step)."""
    from x0ne_core import DecodeMode, Engine, EngineOptions, roofline
    B = args.batch
    prompts = np.stack([splitmix_ids(args.prompt, cfg["vocab_size"], SEED + b) for b in range(B)])
    n_tokens = args.warmup + args.steps + 1
    max_ctx = args.prompt + max(n_tokens, 64) + 16  # room for the oracle fixture's 64 steps too
    t = time.perf_counter()
    e = Engine.load_synthetic(cfg, SEED, STD, EngineOptions(max_ctx=max_ctx, page_seed=1,
                                                            max_batch=B))
    if args.eager:
        e.set_decode_mode(DecodeMode.EAGER)
    print(f"[bench] loaded in {time.perf_counter() - t:.1f} s: {e.describe()}", file=sys.stderr, flush=True)
    runs, tokens = [], None
    for r in range(args.runs):
        toks, secs = e.decode_batch_timed(prompts, args.warmup, args.steps)
        if tokens is None:
            tokens = toks
        elif not (toks == tokens).all():
            raise SystemExit("two runs gave different tokens: the measure is not of one computation")
        runs.append(secs)
        print(f"[bench] run {r}: {B * args.steps / secs:.2f} tok/s ({1e3 * secs / args.steps:.3f} ms per step)",
              file=sys.stderr, flush=True)
    secs = sorted(runs)[len(runs) // 2]
    tok_s = B * args.steps / secs

    # The B prompts to their first tokens (one after the other), twice; the second is reported.
    for _ in range(2):
        _, ptimes = e.greedy_batch(prompts, 1)
    pre_s = float(ptimes[0])
    h, inter, L, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"], cfg["vocab_size"]
    qd, kvd = cfg["num_attention_heads"] * 128, cfg["num_key_value_heads"] * 128
    P = args.prompt
    pre_flops = B * (2 * P * L * (h * (qd + 2 * kvd) + qd * h + 3 * h * inter) + 2 * V * h
                     + 4 * cfg["num_attention_heads"] * 128 * L * (P * (P + 1) // 2))
    prefill = {"tokens": B * P, "seconds": round(pre_s, 6), "tok_s": round(B * P / pre_s, 1),
               "tflops": round(pre_flops / pre_s / 1e12, 2), "peak_tflops": 2500.0,
               "frac": round(pre_flops / pre_s / 1e12 / 2500.0, 4), "flops": pre_flops,
               "timing": "greedy_batch: host time from the call to the first tokens of all sequences"}
    print(f"[bench] prefill {B} x {P} tokens: {pre_s * 1e3:.2f} ms", file=sys.stderr, flush=True)

    shape = roofline.Shape.of(cfg)
    mean_ctx = args.prompt + args.warmup + (args.steps + 1) / 2.0
    step_bytes = roofline.step_bytes(shape, mean_ctx, B)
    hbm_gbs = step_bytes * (args.steps / secs) / 1e9
    # The dominant kernel alone: the batched gate/up projection with SwiGLU behind (weights, the B
    # normed rows in, the B activation rows out).
    gu_bytes = 2 * inter * h * 2 + B * h * 2 + B * inter * 2
    avg_us, wall_us, launches = e.time_kernel("gate_up", args.kernel_iters, batch=B)
    achieved = gu_bytes / (avg_us * 1e-6) / 1e9
    others = {}
    for k in ("qkv", "attention", "o", "down", "head"):
        kus, wus, _ = e.time_kernel(k, args.kernel_iters, batch=B)
        others[k] = {"kernel_us": round(kus, 2), "wall_us": round(wus, 2)}
    others["attention"]["keys_per_sequence"] = e.max_ctx()  # timed at position max_ctx - 1
    print(f"[bench] batched gate_up {avg_us:.2f} us ({achieved:.0f} GB/s), {wall_us:.2f} us per launch with gaps; "
          f"others {others}", file=sys.stderr, flush=True)
    if args.calibrate_copy:
        copy_calibration(args.calibrate_copy << 20)

    # Parity of the timed path: sequence 0's batched greedy tokens against the CPU oracle's
    # committed fixture for its prompt, where one exists. The exact mode has no batched step, so
    # no other mode is timed here.
    fixture = oracle_fixture(args.model, prompts[0])
    timed = {"mode": "f64 sums (exact mode)" if e.exact() else "f32 sums", "tokens_equal_to_oracle": None}
    if fixture is not None:
        n = min(fixture["tokens"].size, tokens.shape[1])
        agree = next((i for i in range(n) if tokens[0][i] != fixture["tokens"][i]), n)
        timed.update({"tokens_equal_to_oracle": agree, "of": n, "source": "batched tokens of sequence 0",
                      "oracle_margin_at_first_difference": None if agree == n else round(fixture["margins"][agree], 6)})
    parity = {"oracle_fixture": fixture["path"] if fixture else None, "timed_path": timed,
              "other_mode": None}
    print(f"[bench] parity {parity['timed_path']}", file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu:
        threads = cpu_threads()
        try:
            cpu = cpu_baseline(cfg, prompts[0], threads, name=model_name)
            cpu["sample"] += "; the oracle decodes one sequence at a time (its tok/s is per sequence)"
        except Exception as ex:
            cpu = {"value": None, "error": str(ex)}
        print(f"[bench] cpu baseline {cpu}", file=sys.stderr, flush=True)
    return {
        "metric": f"{model_name} bf16 decode tok/s @batch{B}; decode HBM GB/s vs 8 TB/s peak",
        "value": round(tok_s, 3), "unit": "tok/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(1e3 * secs / args.steps, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16",
        "data": f"synthetic: random-init N(0,0.02) bf16 weights (seed 0), {B} prompts of uniform random token ids "
                f"(seeds 0..{B - 1})",
        "config": {"workload": f"{model_name}-shape batch-{B} greedy decode of independent prompts, "
                               f"{args.prompt}-token prompts, "
                               + ("eager launches" if args.eager else "hipGraph per batched step"),
                   "batch": B, "layers": L, "hidden": h,
                   "heads": f"{cfg['num_attention_heads']}q/{cfg['num_key_value_heads']}kv", "head_dim": 128,
                   "intermediate": inter, "vocab": V, "tied": cfg["tie_word_embeddings"], "prompt": args.prompt,
                   "mean_ctx": mean_ctx, "runs": runs},
        "decode_hbm": {"achieved": round(hbm_gbs, 1), "peak": 8000.0, "unit": "GB/s",
                       "frac": round(hbm_gbs / 8000.0, 4), "bytes_per_step": int(step_bytes),
                       "ceiling_tok_s": round(roofline.ceiling_tok_s(shape, mean_ctx, B), 2)},
        "roofline": {"kernel": "batched gate_up few-row GEMM (SwiGLU epilogue)", "bound": "hbm",
                     "achieved": round(achieved, 1), "peak": 8000.0, "unit": "GB/s",
                     "frac": round(achieved / 8000.0, 4),
                     "traffic": measured_traffic("batch8 gate_up", BATCH8_TRAFFIC_PROFILE)
                     if (args.model, B) == ("8b", 8) else None,
                     "traffic_source": os.path.relpath(BATCH8_TRAFFIC_PROFILE, ROOT), "bytes_per_launch": gu_bytes,
                     "avg_us": round(avg_us, 3), "wall_us_per_launch": round(wall_us, 3),
                     "launches_timed": launches, "timing": "hipExtLaunchKernel start/stop events per launch",
                     "other_kernels": others},
        "cpu_baseline": cpu,
        "prefill": prefill,
        "tokens_head": tokens[:, :4].tolist(),
    }


FIXTURES = {"8b": "oracle_greedy_8b.json", "0.6b": "oracle_greedy_0_6b.json"}


def oracle_fixture(model: str, prompt: np.ndarray):
    """The CPU oracle's greedy tokens for this workload (tests/golden/make_oracle_greedy.py), when
    one is committed for this shape and prompt."""
    name = FIXTURES.get(model)
    if name is None:
        return None
    path = os.path.join(ROOT, "tests", "golden", name)
    try:
        with open(path) as fh:
            fx = json.load(fh)
    except OSError:
        return None
    if fx["prompt"] != prompt.tolist() or fx["seed"] != SEED or fx["std"] != STD:
        return None
    return {"path": os.path.relpath(path, ROOT), "tokens": np.array(fx["tokens"], np.uint32),
            "margins": fx["margins"]}


def mode_parity(e, prompt, fixture, f64: bool) -> dict:
    """The engine's greedy tokens against the oracle fixture's: how many of the first steps agree,
    and the oracle's top-2 margin where they first differ."""
    out = {"mode": "f64 sums (exact mode)" if f64 else "f32 sums"}
    if fixture is None:
        out["tokens_equal_to_oracle"] = None
        return out
    n = fixture["tokens"].size
    got = e.greedy(prompt, n)
    agree = next((i for i in range(n) if got[i] != fixture["tokens"][i]), n)
    out.update({"tokens_equal_to_oracle": agree, "of": n,
                "oracle_margin_at_first_difference": None if agree == n else round(fixture["margins"][agree], 6)})
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--runs", type=int, default=3, help="timed runs; the median is reported")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU-oracle baseline leg")
    ap.add_argument("--kernel-iters", type=int, default=4)
    ap.add_argument("--eager", action="store_true",
                    help="launch each step's kernels one by one instead of replaying the captured graph "
                         "(for kernel-trace profilers; the same kernels and results)")
    ap.add_argument("--f32-sums", action="store_true",
                    help="time the fp32-accumulating path instead of the engine's default, the exact mode "
                         "(f64 sums in the projections and attention)")
    ap.add_argument("--no-other-mode", action="store_true",
                    help="skip timing the other accumulation mode (the f32 path when the exact mode is timed, "
                         "and back)")
    ap.add_argument("--prompt", type=int, default=PROMPT, help="prompt tokens (config 4: 8192)")
    ap.add_argument("--model", choices=sorted(MODELS), default="8b", help="the Qwen3 shape (default 8b)")
    ap.add_argument("--batch", type=int, default=1,
                    help="independent sequences decoded together (config 4: 8, config 5: 16)")
    ap.add_argument("--attention", action="store_true",
                    help="BASELINE.json config 2 instead: the isolated decode attention at ctx 1k/8k/32k, P 1/4/16")
    ap.add_argument("--attention-iters", type=int, default=64)
    ap.add_argument("--attention-case", default="", metavar="CTX:P",
                    help="--attention at one context and split count only")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="also run one device-to-device copy of MIB MiB (a plain copy kernel of known size, "
                         "for scaling hardware byte counters)")
    args = ap.parse_args()
    # Under rocprofv3 the steps run as eager launches (the same kernels in the same order): a
    # kernel trace over graph replays ended once in a crash inside hipGraphLaunch whose cause was
    # not found, so profiles are taken over eager launches only.
    if not args.eager and (any(k.startswith("ROCPROF") for k in os.environ)
                           or "rocprofiler" in os.environ.get("LD_PRELOAD", "")):
        args.eager = True
        print("[bench] under a profiler: eager launches instead of graph replays", file=sys.stderr, flush=True)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for {args.gpus}); every box here has one, "
              "and no figure at several GPUs is produced. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.attention:
        print(json.dumps(attention_line(args)))
        return
    from x0ne_core import DecodeMode, Engine, EngineOptions, roofline

    model_name, cfg = MODELS[args.model]
    if args.batch > 1:
        print(json.dumps(batch_line(args, model_name, cfg)))
        return
    prompt = splitmix_ids(args.prompt, cfg["vocab_size"], SEED)
    n_tokens = args.warmup + args.steps + 1
    max_ctx = args.prompt + max(n_tokens, 64) + 16  # room for the oracle fixture's 64 steps too
    t = time.perf_counter()
    # The default options (EngineOptions { max_ctx }): the exact mode on this dense batch-1
    # engine; --f32-sums asks for the f32 path.
    e = Engine.load_synthetic(cfg, SEED, STD, EngineOptions(max_ctx=max_ctx, page_seed=1,
                                                            f64_sums=False if args.f32_sums else None))
    exact = e.exact()
    if args.eager:
        e.set_decode_mode(DecodeMode.EAGER)
    load_s = time.perf_counter() - t
    print(f"[bench] loaded in {load_s:.1f} s: {e.describe()}", file=sys.stderr, flush=True)

    runs, tokens = [], None
    for r in range(args.runs):
        toks, secs = e.decode_timed(prompt, args.warmup, args.steps)
        if tokens is None:
            tokens = toks
        elif not (toks == tokens).all():
            raise SystemExit("two runs gave different tokens: the measure is not of one computation")
        runs.append(secs)
        print(f"[bench] run {r}: {args.steps / secs:.2f} tok/s", file=sys.stderr, flush=True)
    secs = sorted(runs)[len(runs) // 2]
    tok_s = args.steps / secs

    # The prompt to its first token, twice (the first also loads code): the second is reported.
    for _ in range(2):
        _, ptimes = e.greedy_timed(prompt, 1)
    pre_s = float(ptimes[0])
    h, inter, L, V = cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"], cfg["vocab_size"]
    qd, kvd = cfg["num_attention_heads"] * 128, cfg["num_key_value_heads"] * 128
    P = args.prompt
    pre_flops = 2 * P * L * (h * (qd + 2 * kvd) + qd * h + 3 * h * inter) + 2 * V * h \
        + 4 * cfg["num_attention_heads"] * 128 * L * (P * (P + 1) // 2)
    pre_peak = 78.6 if exact else 2500.0  # f64 or dense bf16 TFLOP/s of MI355X
    prefill = {"tokens": P, "seconds": round(pre_s, 6), "tok_s": round(P / pre_s, 1),
               "tflops": round(pre_flops / pre_s / 1e12, 2), "peak_tflops": pre_peak,
               "frac": round(pre_flops / pre_s / 1e12 / pre_peak, 4), "flops": pre_flops,
               "timing": "greedy_timed: host time from the call to the first token on the host"}
    print(f"[bench] prefill {P} tokens: {pre_s * 1e3:.2f} ms, {prefill['tok_s']} tok/s, {prefill['tflops']} TFLOP/s",
          file=sys.stderr, flush=True)

    shape = roofline.Shape.of(cfg)
    # Steps w+1..w+K attend prompt + w + 1 .. prompt + w + K positions.
    mean_ctx = args.prompt + args.warmup + (args.steps + 1) / 2.0
    step_bytes = roofline.step_bytes(shape, mean_ctx)
    hbm_gbs = step_bytes * tok_s / 1e9

    # The dominant kernel alone: gate/up GEMV (fused add + RMSNorm in front, SwiGLU behind).
    # Weights, the residual read (f32) and written (f32, block 0), delta and the norm weight (bf16),
    # the SwiGLU output (inter bf16).
    gu_bytes = 2 * inter * h * 2 + 4 * h + 4 * h + 2 * h + 2 * h + 2 * inter
    avg_us, wall_us, launches = e.time_kernel("gate_up", args.kernel_iters)
    achieved = gu_bytes / (avg_us * 1e-6) / 1e9
    others = {}
    for k in ("qkv", "attention", "o", "down", "head"):
        kus, wus, _ = e.time_kernel(k, args.kernel_iters)
        others[k] = {"kernel_us": round(kus, 2), "wall_us": round(wus, 2)}
    others["attention"]["keys"] = e.max_ctx()  # timed at position max_ctx - 1
    print(f"[bench] gate_up {avg_us:.2f} us ({achieved:.0f} GB/s), {wall_us:.2f} us per launch with gaps; "
          f"others {others}", file=sys.stderr, flush=True)

    if args.calibrate_copy:
        copy_calibration(args.calibrate_copy << 20)

    # Parity of the timed path: its greedy tokens against the CPU oracle's committed fixture for
    # this workload (64 steps), and the other accumulation mode timed and checked the same way.
    fixture = oracle_fixture(args.model, prompt)
    parity = {"oracle_fixture": fixture["path"] if fixture else None,
              "timed_path": mode_parity(e, prompt, fixture, exact)}
    if not args.no_other_mode:
        e.close()
        other = Engine.load_synthetic(cfg, SEED, STD, EngineOptions(max_ctx=max_ctx, page_seed=1,
                                                                    f64_sums=not exact))
        if args.eager:
            other.set_decode_mode(DecodeMode.EAGER)
        o_runs = []
        for _ in range(max(1, min(args.runs, 2))):
            o_toks, o_secs = other.decode_timed(prompt, args.warmup, args.steps)
            o_runs.append(o_secs)
        o_secs = min(o_runs)
        o = mode_parity(other, prompt, fixture, not exact)
        compared = min(o_toks.size, tokens.size)
        first_diff = next((i for i in range(compared) if o_toks[i] != tokens[i]), None)
        o.update({"value": round(args.steps / o_secs, 3), "unit": "tok/s", "ms_per_step": round(1e3 * o_secs / args.steps, 4),
                  "decode_hbm_frac": round(step_bytes * args.steps / o_secs / 1e9 / 8000.0, 4),
                  "first_difference_from_timed_path": first_diff,
                  "tokens_compared_with_timed_path": int(compared)})
        parity["other_mode"] = o
        other.close()
        print(f"[bench] other mode {o}", file=sys.stderr, flush=True)
    print(f"[bench] parity {parity['timed_path']}", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu:
        threads = cpu_threads()
        try:
            cpu = cpu_baseline(cfg, prompt, threads, name=model_name)
            if args.model != "0.6b":
                # BASELINE.json config 1 (Qwen3-0.6B, tied, a 20-token prompt, 64 greedy steps) in
                # full: the shape the reference's CPU oracle is quoted on.
                c1 = cpu_baseline(QWEN3_0_6B, prompt[:20], threads, steps=64, prompt_len=min(20, prompt.size),
                                  name="Qwen3-0.6B")
                cpu["config1"] = {k: c1[k] for k in ("value", "unit", "cores", "single_thread_value", "sample")}
        except Exception as ex:  # a baseline that cannot run is reported as missing, not as the GPU's failure
            cpu = {"value": None, "error": str(ex)}
        print(f"[bench] cpu baseline {cpu}", file=sys.stderr, flush=True)

    line = {
        "metric": f"{model_name} bf16 decode tok/s @batch1; decode HBM GB/s vs 8 TB/s peak",
        "value": round(tok_s, 3),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(1e3 * secs / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: random-init N(0,0.02) bf16 weights (seed 0), uniform random token ids (seed 0)",
        "config": {"workload": f"{model_name}-shape batch-1 greedy decode, {args.prompt}-token prompt, "
                               + ("eager launches" if args.eager else "hipGraph per step")
                               + (", exact mode (f64 sums)" if exact else ", f32 sums"),
                   "layers": cfg["num_hidden_layers"], "hidden": cfg["hidden_size"],
                   "heads": f"{cfg['num_attention_heads']}q/{cfg['num_key_value_heads']}kv", "head_dim": 128,
                   "intermediate": cfg["intermediate_size"], "vocab": cfg["vocab_size"],
                   "tied": cfg["tie_word_embeddings"], "prompt": args.prompt, "mean_ctx": mean_ctx, "runs": runs},
        "decode_hbm": {"achieved": round(hbm_gbs, 1), "peak": 8000.0, "unit": "GB/s",
                       "frac": round(hbm_gbs / 8000.0, 4), "bytes_per_step": int(step_bytes),
                       "ceiling_tok_s": round(roofline.ceiling_tok_s(shape, mean_ctx), 2)},
        "roofline": {"kernel": "gate_up GEMV (add+RMSNorm prologue, SwiGLU epilogue)", "bound": "hbm",
                     "achieved": round(achieved, 1), "peak": 8000.0, "unit": "GB/s",
                     "frac": round(achieved / 8000.0, 4), "traffic": measured_traffic("gate_up") if args.model == "8b" else None,
                     "traffic_source": os.path.relpath(TRAFFIC_PROFILE, ROOT), "bytes_per_launch": gu_bytes,
                     "avg_us": round(avg_us, 3), "wall_us_per_launch": round(wall_us, 3),
                     "launches_timed": launches, "timing": "hipExtLaunchKernel start/stop events per launch",
                     "other_kernels": others},
        "cpu_baseline": cpu,
        "prefill": prefill,
        "parity": parity,
        "tokens_head": tokens[:8].tolist(),
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
