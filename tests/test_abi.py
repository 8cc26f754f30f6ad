"""CPU checks of the C-ABI library: it loads, exports every declared entry
point, and its host-side validation mirrors ``Gpu::matmul``'s asserts
(crates/staleynet-cuda/src/ops/matmul.rs:147-149) with distinct codes. No
GPU work is issued here."""
import ctypes
import hashlib
import json
import os
import re

import numpy as np
import pytest

from staleynet_amd import gemm
from staleynet_amd.gemm import BatchStrides, MatmulSpec, Shape, Storage, WriteMode

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    names = []
    for header in sorted(os.listdir(os.path.join(ROOT, "include"))):
        if not header.endswith(".h"):
            continue
        text = open(os.path.join(ROOT, "include", header)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b(sn_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_library_exports_every_declared_entry_point():
    lib = gemm.library()
    names = declared_functions()
    assert "sn_matmul" in names and "sn_matmul_validate" in names and len(names) >= 20
    for name in names:
        assert hasattr(lib, name), f"{name} is declared in include/ but not exported"


def test_every_bound_entry_point_declares_its_argument_types():
    # Without argtypes ctypes passes a Python int as a 32-bit C int: a size_t or pointer parameter
    # then holds whatever the register's upper half held (the planner once read a negative
    # workspace size that way and declined to split K).
    lib = gemm.library()
    bound = sorted(set(re.findall(r'"(sn_[a-z0-9_]+)"', open(gemm.__file__).read())) & set(declared_functions()))
    assert "sn_plan_matmul_column_sums" in bound and len(bound) >= 20
    for name in bound:
        assert getattr(lib, name).argtypes is not None, f"{name} has no argtypes"


def test_spec_new_matches_the_reference_defaults():
    # MatmulSpec::new (ops/matmul.rs:86-97; test :178-188).
    spec = gemm.library().sn_matmul_spec_new(2, 3, 4)
    assert (spec.rows, spec.cols, spec.inner) == (2, 3, 4)
    assert spec.left_storage == 0 and spec.right_storage == 0
    assert (spec.batch_count, spec.batch_left, spec.batch_right, spec.batch_output) == (1, 0, 0, 0)
    assert spec.scale == 1.0 and spec.write == 0 and spec.mask == 0 and spec.precision == 0


def test_python_builders_set_the_expected_fields():
    # ops/matmul.rs:190-207
    spec = (MatmulSpec.new(2, 3, 4).left_transposed().right_transposed().accumulate().scaled(0.25)
            .batched(BatchStrides(count=3, left=8, right=12, output=6)))
    assert spec.left == Storage.Transposed and spec.right == Storage.Transposed
    assert spec.write == WriteMode.Accumulate and spec.scale == 0.25
    assert spec.batch == BatchStrides(3, 8, 12, 6)
    assert BatchStrides.SINGLE == BatchStrides(1, 0, 0, 0)


def test_required_len_accounts_for_the_batch_stride():
    # ops/matmul.rs:209-216
    spec = MatmulSpec.new(2, 3, 4).batched(BatchStrides(count=3, left=8, right=0, output=6))
    assert spec.required_len(8, 8) == 24
    assert spec.required_len(0, 8) == 8
    assert spec.required_len(6, 6) == 18


def test_validate_accepts_exact_lengths_and_reports_each_undersized_operand():
    spec = MatmulSpec.new(5, 7, 3).batched(BatchStrides(count=2, left=15, right=0, output=35))
    left, right, out = spec.lengths()
    assert (left, right, out) == (30, 21, 70)
    assert gemm.validate(spec, left, right, out) == gemm.SN_OK
    assert gemm.validate(spec, left - 1, right, out) == gemm.SN_ERR_LEFT_TOO_SMALL
    assert gemm.validate(spec, left, right - 1, out) == gemm.SN_ERR_RIGHT_TOO_SMALL
    assert gemm.validate(spec, left, right, out - 1) == gemm.SN_ERR_OUTPUT_TOO_SMALL
    # The reference asserts left, then right, then output.
    assert gemm.validate(spec, 0, 0, 0) == gemm.SN_ERR_LEFT_TOO_SMALL


def test_validate_reports_empty_batches_overflow_and_unknown_enums():
    assert gemm.validate(MatmulSpec.new(2, 2, 2).batched(BatchStrides(0, 4, 4, 4)), 99, 99, 99) == \
        gemm.SN_ERR_EMPTY_BATCH
    huge = MatmulSpec.new(1 << 30, 1 << 30, 1 << 30)
    assert gemm.validate(huge, 1 << 62, 1 << 62, 1 << 62) == gemm.SN_ERR_OVERFLOW
    wrap = MatmulSpec.new(2, 2, 2).batched(BatchStrides(3, 1 << 63, 0, 4))
    assert gemm.validate(wrap, 1 << 62, 99, 99) == gemm.SN_ERR_OVERFLOW
    c = MatmulSpec.new(2, 2, 2).to_c()
    c.left_storage = 2
    assert gemm.library().sn_matmul_validate(ctypes.byref(c), 4, 4, 4) == gemm.SN_ERR_UNSUPPORTED
    c = MatmulSpec.new(2, 2, 2).to_c()
    c.mask = 9
    assert gemm.library().sn_matmul_validate(ctypes.byref(c), 4, 4, 4) == gemm.SN_ERR_UNSUPPORTED


def test_zero_sized_products_validate():
    assert gemm.validate(MatmulSpec.new(0, 5, 3), 0, 15, 0) == gemm.SN_OK
    assert gemm.validate(MatmulSpec.new(4, 5, 0), 0, 0, 20) == gemm.SN_OK


def test_null_spec_and_null_context_are_errors_not_crashes():
    lib = gemm.library()
    assert lib.sn_matmul_validate(None, 0, 0, 0) == gemm.SN_ERR_NULL_ARGUMENT
    spec = MatmulSpec.new(1, 1, 1).to_c()
    assert lib.sn_matmul(None, ctypes.byref(spec), None, 1, None, 1, None, 1) == gemm.SN_ERR_NULL_ARGUMENT
    assert lib.sn_synchronize(None) == gemm.SN_ERR_NULL_ARGUMENT
    assert lib.sn_context_destroy(None) == gemm.SN_OK


def test_bias_entry_points_check_lengths_before_touching_the_device():
    # ops/elementwise.rs:33 and :46 assert the vector length against the column count.
    lib = gemm.library()
    assert lib.sn_add_row_bias(None, None, 4, 5, None, 4) == gemm.SN_ERR_LENGTH_MISMATCH
    assert lib.sn_add_row_bias(None, None, 4, 5, None, 5) == gemm.SN_ERR_NULL_ARGUMENT
    assert lib.sn_accumulate_column_sums(None, None, 4, 5, None, 6) == gemm.SN_ERR_LENGTH_MISMATCH
    assert lib.sn_accumulate_column_sums(None, None, 4, 5, None, 5) == gemm.SN_ERR_NULL_ARGUMENT
    spec = MatmulSpec.new(4, 5, 3).to_c()
    assert lib.sn_matmul_bias(None, ctypes.byref(spec), None, 12, None, 15, None, 4, None, 20) == \
        gemm.SN_ERR_LENGTH_MISMATCH
    assert lib.sn_matmul_bias(None, ctypes.byref(spec), None, 11, None, 15, None, 5, None, 20) == \
        gemm.SN_ERR_LEFT_TOO_SMALL
    assert lib.sn_matmul_bias(None, ctypes.byref(spec), None, 12, None, 15, None, 5, None, 20) == \
        gemm.SN_ERR_NULL_ARGUMENT
    shared = MatmulSpec.new(4, 5, 3).batched(gemm.BatchStrides(2, 12, 15, 0)).to_c()
    assert lib.sn_matmul_bias(None, ctypes.byref(shared), None, 24, None, 30, None, 5, None, 20) == \
        gemm.SN_ERR_UNSUPPORTED
    assert gemm.status_string(gemm.SN_ERR_LENGTH_MISMATCH) == "bias or sums length must equal the matrix's columns"


def test_matmul_column_sums_checks_before_touching_the_device():
    # The weight-gradient spec of linear.rs:54-56 with the bias gradient's length check of
    # ops/elementwise.rs:46; only an unbatched product with a row-major right operand is served.
    lib = gemm.library()
    spec = MatmulSpec.new(4, 5, 3).left_transposed().accumulate()
    c = spec.to_c()
    assert lib.sn_matmul_column_sums(None, ctypes.byref(c), None, 11, None, 15, None, 20, None, 5) == \
        gemm.SN_ERR_LEFT_TOO_SMALL
    assert lib.sn_matmul_column_sums(None, ctypes.byref(c), None, 12, None, 15, None, 20, None, 4) == \
        gemm.SN_ERR_LENGTH_MISMATCH
    assert lib.sn_matmul_column_sums(None, ctypes.byref(c), None, 12, None, 15, None, 20, None, 5) == \
        gemm.SN_ERR_NULL_ARGUMENT
    for bad in (spec.right_transposed(), spec.batched(gemm.BatchStrides(2, 12, 15, 20))):
        b = bad.to_c()
        assert lib.sn_matmul_column_sums(None, ctypes.byref(b), None, 24, None, 30, None, 40, None, 5) == \
            gemm.SN_ERR_UNSUPPORTED


def test_row_wise_kernels_check_shapes_before_touching_the_device():
    # ops/attention.rs:59 (rows % queries) and :79 (equal shapes) are asserts in the reference.
    lib = gemm.library()
    assert lib.sn_causal_softmax(None, None, 10, 8, 3, 1.0, 0) == gemm.SN_ERR_SHAPE
    assert lib.sn_causal_softmax(None, None, 10, 8, 0, 1.0, 0) == gemm.SN_ERR_SHAPE
    assert lib.sn_causal_softmax(None, None, 10, 8, 5, 1.0, 0) == gemm.SN_ERR_NULL_ARGUMENT
    assert lib.sn_softmax_backward(None, None, 4, 5, None, 4, 6) == gemm.SN_ERR_SHAPE
    assert lib.sn_softmax_backward(None, None, 4, 5, None, 4, 5) == gemm.SN_ERR_NULL_ARGUMENT


def test_cross_entropy_checks_before_touching_the_device():
    # ops/loss.rs:44-47: gradient shape, head inside the row, losses and targets long enough.
    lib = gemm.library()
    head = gemm.CCrossEntropyHead(10, 37, 2, 1, 0.25)
    args = lambda rows, targets, losses, grows, gcols: (None, None, rows, 50, None, targets, ctypes.byref(head),  # noqa
                                                        None, losses, None, grows, gcols)
    assert lib.sn_cross_entropy(*args(13, 26, 13, 13, 49)) == gemm.SN_ERR_SHAPE
    assert lib.sn_cross_entropy(None, None, 13, 46, None, 26, ctypes.byref(head), None, 13, None, 13, 46) == \
        gemm.SN_ERR_SHAPE
    assert lib.sn_cross_entropy(*args(13, 26, 12, 13, 50)) == gemm.SN_ERR_LENGTH_MISMATCH
    assert lib.sn_cross_entropy(*args(13, 25, 13, 13, 50)) == gemm.SN_ERR_LENGTH_MISMATCH
    assert lib.sn_cross_entropy(*args(13, 26, 13, 13, 50)) == gemm.SN_ERR_NULL_ARGUMENT


def test_status_strings_carry_the_reference_panic_messages():
    assert gemm.status_string(gemm.SN_ERR_LEFT_TOO_SMALL) == "matmul: left operand too small"
    assert gemm.status_string(gemm.SN_ERR_RIGHT_TOO_SMALL) == "matmul: right operand too small"
    assert gemm.status_string(gemm.SN_ERR_OUTPUT_TOO_SMALL) == "matmul: output too small"
    for code in range(-12, 1):
        assert gemm.status_string(code)


def test_kernel_tolerances_follow_the_reference_convention():
    assert gemm.MatmulKernel.MfmaF32.tolerance() == pytest.approx(1e-5)
    assert gemm.MatmulKernel.Simple.tolerance() == pytest.approx(1e-5)
    assert gemm.MatmulKernel.MfmaBf16.tolerance() == pytest.approx(2e-2)


def test_shape_helpers():
    assert len(Shape.new(3, 4)) == 12 and Shape.vector(5) == Shape(1, 5)


def test_oracle_reproduces_the_committed_sweep_vectors():
    # The same vectors the GPU tests compare against; a change in the oracle build shows here first.
    from oracle import oracle
    import sys
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    import make_golden

    golden = json.load(open(os.path.join(ROOT, "tests", "golden", "sweep_oracle.json")))["cases"]
    for record in golden:
        out = make_golden.oracle_output(record)
        assert hashlib.sha256(out.astype("<f4").tobytes()).hexdigest() == record["sha256"]
        assert out[:8].tolist() == record["first"]


def test_context_creation_without_a_gpu_fails_cleanly():
    lib = gemm.library()
    count = ctypes.c_int(0)
    hip = ctypes.CDLL("libamdhip64.so")
    if hip.hipGetDeviceCount(ctypes.byref(count)) == 0 and count.value > 0:
        pytest.skip("a GPU is present")
    handle = ctypes.c_void_p()
    assert lib.sn_context_create(0, ctypes.byref(handle)) == gemm.SN_ERR_NO_DEVICE
    assert not handle.value


def test_struct_layouts_match_the_header():
    # The layouts a Rust #[repr(C)] binding mirrors (LP64): sizes and the offsets after each
    # 4-byte field, where padding would show up. context.cpp pins the same with static_assert.
    spec = gemm.CMatmulSpec
    assert ctypes.sizeof(spec) == 88
    assert [spec.left_storage.offset, spec.batch_count.offset, spec.scale.offset, spec.write.offset,
            spec.mask.offset, spec.precision.offset, spec.query_offset.offset] == [24, 32, 64, 68, 72, 76, 80]
    shape = gemm.CAttentionShape
    assert ctypes.sizeof(shape) == 64 and shape.query_offset.offset == 48 and shape.scale.offset == 56
    layout = gemm.CHeadLayout
    assert ctypes.sizeof(layout) == 64 and layout.time_offset.offset == 56
    head = gemm.CCrossEntropyHead
    assert ctypes.sizeof(head) == 40 and head.grad_scale.offset == 32
    plan = gemm.CLaunchPlan
    assert ctypes.sizeof(plan) == 72 and plan.k_per_split.offset == 32 and plan.workspace_bytes.offset == 64
