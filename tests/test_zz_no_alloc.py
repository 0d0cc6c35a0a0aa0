"""The split-K decode attention's no-allocation entry point (x0ne_gpu_attention_split_scratch:
its states and counters in the library's static scratch array) against the entry point that
takes them as workspace arguments (x0ne_gpu_attention_split): the same bits, on two calls in a
row, the second with a smaller input (fewer heads, fewer keys, another P), with either merge;
and the refusal of a geometry past the array's size."""
import numpy as np
import pytest

from common import O, bf16_bits

pytestmark = pytest.mark.gpu


def H(q, kv):
    from x0ne_core.ops import Heads
    return Heads(q, kv)


@pytest.mark.parametrize("last_block", [True, False])
def test_the_scratch_entry_point_gives_the_workspace_entry_points_bits(kernels, last_block):
    rng = O.Rng(880 + int(last_block))
    for qh, kvh, ctx, splits in [(32, 8, 4097, None), (8, 2, 300, 4), (64, 8, 1000, 16)]:
        h = H(qh, kvh)
        q = bf16_bits(rng.bf16s(h.q_dim, 3.0))
        k = bf16_bits(rng.bf16s(ctx * h.kv_dim, 1.0))
        v = bf16_bits(rng.bf16s(ctx * h.kv_dim, 4.0))
        pages = (ctx + 15) // 16
        page_of = [int(p) for p in np.random.default_rng(ctx).permutation(pages + 3)[:pages]]
        want = kernels.attention_decode_split(q, k, v, ctx, h, last_block=last_block, splits=splits,
                                              page_of=page_of)
        got = kernels.attention_decode_split_scratch(q, k, v, ctx, h, last_block=last_block, splits=splits,
                                                     page_of=page_of)
        assert (got == want).all(), f"{qh}/{kvh} ctx {ctx} P {splits}: {int((got != want).sum())} outputs differ"
        again = kernels.attention_decode_split_scratch(q, k, v, ctx, h, last_block=last_block, splits=splits,
                                                       page_of=page_of)
        assert (again == want).all(), f"{qh}/{kvh} ctx {ctx}: a repeated call"
        print(f"MEASURE scratch split-K {qh}/{kvh} ctx {ctx} P {splits} last_block {last_block}: bit-equal")


def test_a_geometry_past_the_scratch_array_is_refused(kernels):
    from x0ne_core import FormatError
    g = kernels.gpu
    plan = g.split_plan(64, 8)
    plan.splits = 256  # 64 heads x 256 slices x 528 bytes = 8.65 MB of states > 4 MiB
    with pytest.raises(FormatError, match="scratch"):
        g.attention_split_scratch(plan, True, 16, 16, 16, 16, 16, 16, 64, 8, 1024, 0.088)
    plan = g.split_plan(257, 257)
    plan.splits = 1  # 257 counters > 256
    with pytest.raises(FormatError, match="scratch"):
        g.attention_split_scratch(plan, True, 16, 16, 16, 16, 16, 16, 257, 257, 1024, 0.088)
