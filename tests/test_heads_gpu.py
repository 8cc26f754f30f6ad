"""GPU parity of the attention head permutes (``sn_split_heads`` / ``sn_merge_heads``,
``Gpu::split_heads`` / ``merge_heads``, ops/attention.rs:20-52): bit-exact against the oracle's
restatement of kernels/attention.rs:77-138. The reference's own GPU test
(tests/kernels_match_reference.rs:199-231) comes first, on its inputs; then config 3's QKV
split and merge, a cache append, the scalar (unaligned) path and the layout checks.
"""
import numpy as np
import pytest

from oracle import oracle
from staleynet_amd.gemm import HeadLayout, Shape

pytestmark = pytest.mark.gpu


def to_oracle(layout: HeadLayout) -> oracle.HeadLayout:
    return oracle.HeadLayout(layout.batch, layout.time, layout.heads, layout.head_dim, layout.width,
                             layout.column_offset, layout.time_capacity, layout.time_offset)


def check_split_and_merge(gpu, layout, packed, seed):
    major_len = layout.batch * layout.heads * layout.time_capacity * layout.head_dim
    initial = oracle.random_values(major_len, seed)  # untouched steps of the head-major buffer keep their values
    P = gpu.upload(Shape(layout.batch * layout.time, layout.width), packed)
    M = gpu.upload(Shape.vector(major_len), initial)
    gpu.split_heads(P, M, layout)
    expected = initial.copy()
    oracle.split_heads(packed, expected, to_oracle(layout))
    assert np.array_equal(gpu.download(M), expected)
    base = oracle.random_values(packed.size, seed + 1)
    Q = gpu.upload(Shape(layout.batch * layout.time, layout.width), base)
    gpu.merge_heads(M, Q, layout)
    expected_packed = base.copy()
    oracle.merge_heads(expected, expected_packed, to_oracle(layout))
    assert np.array_equal(gpu.download(Q), expected_packed)


def test_reference_split_and_merge_test(gpu):
    layout = HeadLayout.dense(2, 5, 3, 4, 3 * 12 + 2, 13).in_cache(9, 2)
    packed = oracle.random_values(layout.batch * layout.time * layout.width, 12)
    P = gpu.upload(Shape(layout.batch * layout.time, layout.width), packed)
    M = gpu.zeros(Shape(layout.batch * layout.heads * layout.time_capacity, layout.head_dim))
    gpu.split_heads(P, M, layout)
    split = gpu.download(M)
    for b in range(2):
        for h in range(3):
            for t in range(5):
                for d in range(4):
                    assert split[((b * 3 + h) * 9 + 2 + t) * 4 + d] == packed[(b * 5 + t) * layout.width + 13 + h * 4 + d]
    merged = gpu.zeros(Shape(layout.batch * layout.time, layout.width))
    gpu.merge_heads(M, merged, layout)
    columns = np.arange(packed.size) % layout.width
    inside = (columns >= 13) & (columns < 13 + 12)
    assert np.array_equal(gpu.download(merged), np.where(inside, packed, 0.0).astype(np.float32))


@pytest.mark.parametrize("part", [0, 1, 2])
def test_config_3_qkv_split_and_merge(gpu, part):
    # 2 of config 3's 16 sequences: packed QKV [2 x 2048, 3 x 768], 12 heads of 64, Q/K/V at offsets 0/768/1536.
    batch, time, heads, head_dim = 2, 2048, 12, 64
    width = 3 * heads * head_dim
    layout = HeadLayout.dense(batch, time, heads, head_dim, width, part * heads * head_dim)
    check_split_and_merge(gpu, layout, oracle.random_values(batch * time * width, 40 + part), 50 + part)


def test_cache_append_of_one_step(gpu):
    # Decode: one new position's keys into a 1408-step cache at step 700 (layers/attention.rs:288-297).
    layout = HeadLayout.dense(1, 1, 12, 64, 3 * 768, 768).in_cache(1408, 700)
    check_split_and_merge(gpu, layout, oracle.random_values(3 * 768, 60), 61)


def test_unaligned_layout_takes_the_scalar_path(gpu):
    layout = HeadLayout.dense(3, 7, 5, 3, 17, 1).in_cache(11, 4)
    check_split_and_merge(gpu, layout, oracle.random_values(3 * 7 * 17, 62), 63)


def test_layout_checks_raise_the_reference_panics(gpu):
    packed, major = gpu.zeros(Shape(10, 24)), gpu.zeros(Shape(2 * 3 * 5, 4))
    with pytest.raises(AssertionError, match="HeadLayout: time range exceeds capacity"):
        gpu.split_heads(packed, major, HeadLayout.dense(2, 5, 3, 4, 24, 0).in_cache(5, 1))
    with pytest.raises(AssertionError, match="HeadLayout: packed tensor too small"):
        gpu.split_heads(packed, major, HeadLayout.dense(2, 6, 3, 4, 24, 0))
    with pytest.raises(AssertionError, match="HeadLayout: head-major tensor too small"):
        gpu.split_heads(packed, major, HeadLayout.dense(2, 5, 3, 4, 24, 0).in_cache(6, 0))
