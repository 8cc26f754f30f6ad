"""GPU test of sn_matmul_noalloc, the allocation-free variant of sn_matmul (its scratch is a device
array of the library's, not a context's workspace): on the same inputs it must give sn_matmul's
result, bit for bit where both plan the same launch (the planner tells), else within the fp32
tolerance. Each case is two calls in a row on one device, the second on a smaller input, so the
second call runs on the scratch (counters and partial sums) the first one left; fp32 and bf16.

Graph capture, the use the header names: in a fresh process, the first calls on the device (the
ones that look up the scratch's address) are made under stream capture, in global and in relaxed
capture mode; the graph is replayed three times with eager calls and synchronizations between the
replays, and every replay must equal sn_matmul's eager result."""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import oracle  # noqa: E402
from staleynet_amd import gemm  # noqa: E402
from staleynet_amd.gemm import MatmulSpec, Precision, Shape  # noqa: E402

pytestmark = pytest.mark.gpu

TOLERANCE = 1e-5  # kernels_match_reference.rs:12


def noalloc_status(gpu, spec, left, right, out):
    c = spec.to_c()
    return gemm.library().sn_matmul_noalloc(ctypes.byref(c), ctypes.c_void_p(left.pointer), len(left),
                                            ctypes.c_void_p(right.pointer), len(right), ctypes.c_void_p(out.pointer),
                                            len(out), ctypes.c_void_p(gpu.stream))


def noalloc(gpu, spec, left, right, out):
    rc = noalloc_status(gpu, spec, left, right, out)
    assert rc == gemm.SN_OK, gemm.status_string(rc)


def same_launch(spec):
    """Whether sn_matmul (a context's 1.5 GiB workspace) and sn_matmul_noalloc (its 64 MiB) plan the
    same launch, which then sums in the same order."""
    a, b = gemm.plan(spec), gemm.plan(spec, workspace_bytes=64 << 20)
    return (a.path, a.splits, a.k_per_split, a.tile_rows, a.tile_cols) == \
        (b.path, b.splits, b.k_per_split, b.tile_rows, b.tile_cols)


def agree(spec, expected, got):
    """sn_matmul_noalloc's result against sn_matmul's: the same bits for the same launch, else within
    the fp32 tolerance (both round the same operands the same way; only the summation order differs)."""
    assert np.all(np.isfinite(got))
    if same_launch(spec):
        assert np.array_equal(expected, got)
    else:
        assert oracle.relative_error(expected, got) < TOLERANCE


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
    agree(spec, expected, got)


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
    # bf16 inputs: a forward product, then a split weight gradient.
    (MatmulSpec.new(1024, 2304, 768).with_precision(Precision.Bf16),
     MatmulSpec.new(768, 768, 8192).left_transposed().accumulate().with_precision(Precision.Bf16)),
    # bf16 on a head-sized weight gradient (staged operands would not fit the scratch), then NT.
    (MatmulSpec.new(768, 16384, 2048).left_transposed().accumulate().with_precision(Precision.Bf16),
     MatmulSpec.new(512, 768, 2304).right_transposed().with_precision(Precision.Bf16)),
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


# Products captured on the first calls of a fresh process: split K with arrival counters (decode),
# split-K partial sums (weight gradient), and bf16 (a forward product and a split weight gradient).
CAPTURED = [
    MatmulSpec.new(1, 2304, 768),
    MatmulSpec.new(4, 768, 3072).accumulate(),
    MatmulSpec.new(256, 256, 8192).left_transposed().accumulate(),
    MatmulSpec.new(512, 768, 1024).with_precision(Precision.Bf16),
    MatmulSpec.new(768, 768, 4096).left_transposed().accumulate().with_precision(Precision.Bf16),
]


def capture_child(mode: int) -> None:
    """Runs in a fresh process: nothing calls sn_matmul_noalloc before the capture."""
    from bench import hip_runtime

    gpu = gemm.Gpu(0)
    hip = hip_runtime()
    stream = ctypes.c_void_p(gpu.stream)
    cases = []
    for i, spec in enumerate(CAPTURED):
        left_len, right_len, out_len = spec.lengths()
        left = gpu.upload(Shape.vector(left_len), oracle.random_values(left_len, 70 + 3 * i))
        right = gpu.upload(Shape.vector(right_len), oracle.random_values(right_len, 71 + 3 * i))
        initial = oracle.random_values(out_len, 72 + 3 * i)
        cases.append((spec, left, right, gpu.upload(Shape.vector(out_len), initial), initial))
    gpu.synchronize()
    print(f"capture mode {mode}: begin", flush=True)
    assert hip.hipStreamBeginCapture(stream, mode) == 0
    statuses = [noalloc_status(gpu, spec, left, right, out) for spec, left, right, out, _ in cases]
    graph = ctypes.c_void_p()
    end = hip.hipStreamEndCapture(stream, ctypes.byref(graph))
    assert statuses == [gemm.SN_OK] * len(cases), [gemm.status_string(rc) for rc in statuses]
    assert end == 0, f"hipStreamEndCapture: {end}"
    executable = ctypes.c_void_p()
    assert hip.hipGraphInstantiate(ctypes.byref(executable), graph, None, None, ctypes.c_size_t(0)) == 0
    try:
        # The capture ran nothing: the outputs still hold their initial values.
        for spec, _, _, out, initial in cases:
            assert np.array_equal(gpu.download(out), initial), "a captured call ran eagerly"
        expected = []
        for spec, left, right, _, initial in cases:
            reference_out = gpu.upload(Shape.vector(initial.size), initial)
            gpu.matmul(spec, left, right, reference_out)
            expected.append(gpu.download(reference_out))
            reference_out.free()
        small = MatmulSpec.new(2, 768, 768)
        x = gpu.upload(Shape.vector(2 * 768), oracle.random_values(2 * 768, 90))
        w = gpu.upload(Shape.vector(768 * 768), oracle.random_values(768 * 768, 91))
        y, y_ref = gpu.zeros(Shape.vector(2 * 768)), gpu.zeros(Shape.vector(2 * 768))
        gpu.matmul(small, x, w, y_ref)
        for replay in range(3):
            for _, _, _, out, initial in cases:
                gpu.copy_from_host(out, initial)
            assert hip.hipGraphLaunch(executable, stream) == 0
            gpu.synchronize()
            for (spec, _, _, out, _), want in zip(cases, expected):
                agree(spec, want, gpu.download(out))
            # Eager allocation-free and context calls between the replays, on the same scratch.
            noalloc(gpu, small, x, w, y)
            gpu.matmul(MatmulSpec.new(1, 768, 768), x, w, gpu.zeros(Shape.vector(768)))
            gpu.synchronize()
            agree(small, gpu.download(y_ref), gpu.download(y))
            print(f"capture mode {mode}: replay {replay} matches", flush=True)
    finally:
        hip.hipGraphExecDestroy(executable)
        hip.hipGraphDestroy(graph)
    gpu.close()


@pytest.mark.parametrize("mode", [0, 2], ids=["global_capture", "relaxed_capture"])
def test_first_calls_under_graph_capture_replay_like_sn_matmul(mode):
    print(f"noalloc capture in a fresh process, mode {mode}", flush=True)
    proc = subprocess.run([sys.executable, os.path.abspath(__file__), "capture", str(mode)], cwd=ROOT,
                          stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=240)
    print(proc.stdout[-4000:])
    assert proc.returncode == 0


if __name__ == "__main__" and len(sys.argv) == 3 and sys.argv[1] == "capture":
    capture_child(int(sys.argv[2]))
