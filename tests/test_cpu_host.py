"""Host-side logic without a GPU: the roofline formula against the reference's published ceiling,
the bench's workload generator against the oracle's, and the host metrics against the oracle's."""
import sys

import numpy as np

from common import O, ROOT


def test_the_roofline_reproduces_the_references_h100_ceiling_and_the_mi355x_targets():
    """roofline.rs:55-102; the published 221.13 tok/s H100 ceiling of Qwen3-8B at prompt 20 and
    256 generated (3,352 GB/s), and the 8 TB/s targets of the decode configs."""
    from x0ne_core import roofline
    from bench import QWEN3_8B
    s = roofline.Shape.of(QWEN3_8B)
    # 2 [36 (4096 * 6144 + 4096 * 4096 + 3 * 4096 * 12288 + 2 * 4096 + 2 * 128) + 4096 + 151936 * 4096 + 4096]
    assert roofline.weight_bytes_per_token(s) == 2 * (36 * 192946432 + 622338048) == 15136819200
    assert roofline.kv_bytes_per_position(s) == 147456
    ctx = roofline.mean_decode_ctx(20, 256)
    assert abs(roofline.ceiling_tok_s(s, ctx, bandwidth_gbs=3352.0) - 221.13) < 0.01
    assert abs(roofline.ceiling_tok_s(s, ctx) - 527.8) < 0.05
    assert abs(roofline.ceiling_tok_s(s, roofline.mean_decode_ctx(8192, 512)) - 488.3) < 0.05
    assert abs(roofline.ceiling_tok_s(s, roofline.mean_decode_ctx(8192, 512), batch=8) - 2549.5) < 0.1
    s32 = roofline.Shape(5120, 25600, 64, 64, 8, 128, 151936)
    assert abs(roofline.ceiling_tok_s(s32, roofline.mean_decode_ctx(512, 256)) - 124.7) < 0.05


def test_the_bench_prompt_is_the_oracles_splitmix_stream():
    import bench
    assert (bench.splitmix_ids(20, 151936, 0) == O.synthetic_ids(20, 151936, 0)).all()
    # The reference's known answer (bench_tests.rs:1072-1081).
    assert bench.splitmix_ids(6, 151936, 0x0C0E5EED).tolist() == [126819, 135692, 59481, 30850, 145817, 72711]


def test_the_bench_refuses_more_than_one_gpu():
    import subprocess
    r = subprocess.run([sys.executable, f"{ROOT}/bench.py", "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0 and "one GPU" in r.stderr


def test_host_metrics_are_the_oracles():
    from x0ne_core import metrics
    rng = np.random.default_rng(0)
    for _ in range(20):
        p = rng.normal(0, 3, 1000).astype(np.float32)
        q = (p + rng.normal(0, 0.1, 1000)).astype(np.float32)
        assert metrics.argmax(p) == O.argmax(p)
        assert abs(metrics.logsumexp(p) - O.logsumexp(p)) < 1e-12 * abs(O.logsumexp(p))
        assert abs(metrics.kl(p, q) - O.kl(p, q)) < 1e-12
    assert metrics.argmax([1.0, float("nan")]) is None and O.argmax([1.0, float("nan")]) is None
    assert metrics.argmax([2.0, 2.0]) == 0


def test_panel_layout_round_trips_and_places_each_element():
    """The batched step's X layout (ops.to_panels): element (t, k) of [n][cols] at
    ((t / 16 * cols / 8 + k / 8) * 16 + t % 16) * 8 + k % 8, rows past n zero."""
    import numpy as np
    from x0ne_core.ops import from_panels, to_panels
    for n, cols in [(1, 8), (16, 8), (17, 24), (40, 4096)]:
        m = np.arange(n * cols, dtype=np.uint32).reshape(n, cols) + 1
        p = to_panels(m)
        assert p.size == -(-n // 16) * 16 * cols and (p != 0).sum() == n * cols
        for t, k in [(0, 0), (n - 1, cols - 1), (n // 2, cols // 3)]:
            assert p[(((t // 16) * (cols // 8) + k // 8) * 16 + t % 16) * 8 + k % 8] == m[t, k]
        assert (from_panels(p, n, cols) == m).all()


def test_the_exact_attention_without_a_last_block_merge_is_refused_before_any_device_work():
    """The exact decode attention has no f64 merge kernel behind it, so the helper refuses
    last_block=False before it plans, allocates or launches anything: the stub device below
    raises on any use."""
    import pytest
    from x0ne_core import FormatError
    from x0ne_core.ops import Heads, Kernels

    class NoDevice:
        def __getattr__(self, name):
            raise AssertionError(f"device touched: {name}")

    h = Heads(4, 2, 128)
    ctx = 5
    qkv = np.zeros(h.q_dim + 2 * h.kv_dim, np.uint16)
    kv = np.zeros((ctx - 1) * h.kv_dim, np.uint16)
    norm = np.zeros(128, np.uint16)
    with pytest.raises(FormatError, match="last block"):
        Kernels(NoDevice()).attention_rope_decode(qkv, norm, norm, 1e-6, 1e6, kv, kv, ctx, h, last_block=False,
                                                  exact=True)
