"""GPU test of sn_matmul_noalloc, the allocation-free variant of sn_matmul (its scratch is a device
array of the library's, not a context's workspace): on the same inputs it must give sn_matmul's
result, bit for bit where both plan the same split of K (the planner tells), else within the fp32
tolerance. Each case is two calls in a row on one device, the second on a smaller input, so the
second call runs on the scratch (counters and partial sums) the first one left."""
import ctypes

import numpy as np
import pytest

from oracle import oracle
from staleynet_amd import gemm
from staleynet_amd.gemm import MatmulSpec, Shape

pytestmark = pytest.mark.gpu

TOLERANCE = 1e-5  # kernels_match_reference.rs:12


def noalloc(gpu, spec, left, right, out):
    c = spec.to_c()
    rc = gemm.library().sn_matmul_noalloc(ctypes.byref(c), ctypes.c_void_p(left.pointer), len(left),
                                          ctypes.c_void_p(right.pointer), len(right), ctypes.c_void_p(out.pointer),
                                          len(out), ctypes.c_void_p(gpu.stream))
    assert rc == gemm.SN_OK, gemm.status_string(rc)


def compare(gpu, spec, seed):
    """sn_matmul and sn_matmul_noalloc on the same seeded operands and initial output."""
    left_len, right_len, out_len = spec.lengths()
    left = gpu.upload(Shape.vector(left_len), oracle.random_values(left_len, seed))
    right = gpu.upload(Shape.vector(right_len), oracle.random_values(right_len, seed + 1))
    initial = oracle.random_values(out_len, seed + 2)
    reference_out = gpu.upload(Shape.vector(out_len), initial)
    static_out = gpu.upload(Shape.vector(out_len), initial)
    gpu.matmul(spec, left, right, reference_out)
    noalloc(gpu, spec, left, right, static_out)
    expected, got = gpu.download(reference_out), gpu.download(static_out)
    for t in (left, right, reference_out, static_out):
        t.free()
    assert np.all(np.isfinite(got))
    same_plan = gemm.plan(spec).splits == gemm.plan(spec, workspace_bytes=64 << 20).splits
    if same_plan:
        assert np.array_equal(expected, got)
    else:
        assert oracle.relative_error(expected, got) < TOLERANCE
    return same_plan


@pytest.mark.parametrize("first,second", [
    # Decode products (split K, partial sums and arrival counters in the scratch): qkv, then out.
    (MatmulSpec.new(1, 2304, 768), MatmulSpec.new(1, 768, 768)),
    # Four rows, accumulating: up, then down.
    (MatmulSpec.new(4, 3072, 768).accumulate(), MatmulSpec.new(4, 768, 3072).accumulate()),
    # Weight gradients with split K (TN, accumulate), the second smaller.
    (MatmulSpec.new(256, 256, 8192).left_transposed().accumulate(),
     MatmulSpec.new(128, 128, 4096).left_transposed().accumulate()),
    # A head-sized weight gradient whose partial sums would exceed the scratch: fewer slices.
    (MatmulSpec.new(768, 16384, 4096).left_transposed().accumulate(),
     MatmulSpec.new(768, 2304, 4096).left_transposed().accumulate()),
])
def test_noalloc_matches_sn_matmul_on_two_calls_in_a_row(gpu, first, second):
    print(f"noalloc: {first.rows}x{first.cols}x{first.inner} then {second.rows}x{second.cols}x{second.inner}",
          flush=True)
    compare(gpu, first, 11)
    compare(gpu, second, 21)
    gpu.synchronize()


def test_noalloc_checks_like_sn_matmul(gpu):
    spec = MatmulSpec.new(4, 4, 4)
    small = gpu.zeros(Shape.vector(8))
    ok = gpu.zeros(Shape.vector(16))
    c = spec.to_c()
    lib = gemm.library()
    rc = lib.sn_matmul_noalloc(ctypes.byref(c), ctypes.c_void_p(small.pointer), 8, ctypes.c_void_p(ok.pointer), 16,
                               ctypes.c_void_p(ok.pointer), 16, None)
    assert rc == gemm.SN_ERR_LEFT_TOO_SMALL
    other = gpu.zeros(Shape.vector(16))
    rc = lib.sn_matmul_noalloc(ctypes.byref(c), ctypes.c_void_p(ok.pointer), 16, ctypes.c_void_p(other.pointer), 16,
                               ctypes.c_void_p(ok.pointer), 16, None)
    assert rc == gemm.SN_ERR_ALIASING
    for t in (small, ok, other):
        t.free()
