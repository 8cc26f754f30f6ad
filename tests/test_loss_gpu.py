"""GPU parity of the per-codebook cross-entropy (``sn_cross_entropy``, ``Gpu::cross_entropy``,
ops/loss.rs:34-71) against the oracle's ``reference::cross_entropy`` (reference.rs:139-166).

The reference's own GPU test (tests/kernels_match_reference.rs:277-298) comes first, on its
inputs; then the reference's CPU known-answer cases on the device, the register-resident and
multi-pass paths, config 2's 16-codebook head at scale (every codebook, as training.rs:208-239
calls it), and the shape checks.
"""
import numpy as np
import pytest

from oracle import oracle
from staleynet_amd.gemm import EMPTY_TOKEN, CrossEntropyHead, Shape

pytestmark = pytest.mark.gpu

TOLERANCE = 1e-5  # kernels_match_reference.rs:12


def run(gpu, logits, targets, rows, cols, head, grad_init=None):
    grad_init = np.zeros(rows * cols, np.float32) if grad_init is None else grad_init
    L = gpu.upload(Shape(rows, cols), logits)
    T = gpu.upload_tokens(targets)
    losses = gpu.zeros(Shape.vector(rows))
    grad = gpu.upload(Shape(rows, cols), grad_init)
    gpu.cross_entropy(L, T, head, losses, grad)
    expected_losses = np.zeros(rows, np.float32)
    expected_grad = grad_init.copy()
    oracle.cross_entropy(logits, targets, cols,
                         oracle.CrossEntropyHead(head.column_offset, head.classes, head.target_stride,
                                                 head.target_offset, head.grad_scale),
                         expected_losses, expected_grad)
    return expected_losses, gpu.download(losses), expected_grad, gpu.download(grad)


def test_reference_cross_entropy_gpu_test(gpu):
    rows, cols = 13, 50
    head = CrossEntropyHead(column_offset=10, classes=37, target_stride=2, target_offset=1, grad_scale=0.25)
    logits = oracle.random_values(rows * cols, 15)
    targets = np.array([EMPTY_TOKEN if i % 7 == 0 else (i * 5 % head.classes) for i in range(rows * 2)], np.uint32)
    el, gl, eg, gg = run(gpu, logits, targets, rows, cols, head)
    assert oracle.relative_error(el, gl) < TOLERANCE
    assert oracle.relative_error(eg, gg) < TOLERANCE


def test_reference_known_answers_on_the_device(gpu):
    head = CrossEntropyHead(0, 3, 1, 0, 1.0)
    logits = np.array([1, 2, 3, 0, 0, 0, 0, 0], np.float32)
    el, gl, eg, gg = run(gpu, logits, np.array([2, 0], np.uint32), 2, 4, head, np.full(8, 7.0, np.float32))
    assert gl == pytest.approx([0.407606, 1.098612], abs=1e-5)
    assert gg[3] == 7.0 and gg[7] == 7.0  # columns outside the head are left alone
    assert oracle.relative_error(eg, gg) < TOLERANCE
    el, gl, eg, gg = run(gpu, logits, np.array([EMPTY_TOKEN, 0], np.uint32), 2, 4, head, np.full(8, 7.0, np.float32))
    assert gl[0] == 0.0 and gg[:3].tolist() == [0.0, 0.0, 0.0] and gg[3] == 7.0


@pytest.mark.parametrize("rows,cols,offset,classes,stride,toff,scale", [
    (64, 1024, 0, 1024, 1, 0, 1.0),          # one codebook, aligned: register-resident
    (33, 4096, 1024, 1024, 4, 3, 0.0625),    # a codebook in a 4-codebook row
    (20, 5000, 0, 4600, 1, 0, 0.5),          # past 4096 classes: multi-pass
    (17, 101, 3, 97, 2, 1, 0.125),           # unaligned: multi-pass
    (8, 16384, 15360, 1024, 16, 15, 1 / 128),  # the last of 16 codebooks
])
def test_cross_entropy_matches_the_oracle(gpu, rows, cols, offset, classes, stride, toff, scale):
    rng = np.random.default_rng(rows + cols)
    logits = rng.normal(0, 2, rows * cols).astype(np.float32)
    targets = rng.integers(0, classes, rows * stride).astype(np.uint32)
    targets[::5] = EMPTY_TOKEN
    head = CrossEntropyHead(offset, classes, stride, toff, scale)
    el, gl, eg, gg = run(gpu, logits, targets, rows, cols, head, rng.normal(0, 1, rows * cols).astype(np.float32))
    assert oracle.relative_error(el, gl) < TOLERANCE
    assert oracle.relative_error(eg, gg) < TOLERANCE


def test_config_2_head_every_codebook(gpu):
    # 2048 of config 2's 32768 rows, logits [2048, 16 x 1024] ~N(0, 1), 16 codebooks as training.rs calls them.
    rows, codebooks, size = 2048, 16, 1024
    cols = codebooks * size
    logits = gpu.zeros(Shape(rows, cols))
    gpu.fill_normal(logits, 1234, 31)
    host_logits = gpu.download(logits)
    rng = np.random.default_rng(9)
    targets = rng.integers(0, size, rows * codebooks).astype(np.uint32)
    targets[rng.random(rows * codebooks) < 0.02] = EMPTY_TOKEN
    T = gpu.upload_tokens(targets)
    grad = gpu.zeros(Shape(rows, cols))
    losses = gpu.zeros(Shape.vector(rows))
    expected_grad = np.zeros(rows * cols, np.float32)
    for c in range(codebooks):
        valid = int(np.sum(targets[c::codebooks] != EMPTY_TOKEN))
        head = CrossEntropyHead(c * size, size, codebooks, c, 1.0 / (valid * codebooks))
        gpu.cross_entropy(logits, T, head, losses, grad)
        expected_losses = np.zeros(rows, np.float32)
        oracle.cross_entropy(host_logits, targets, cols,
                             oracle.CrossEntropyHead(c * size, size, codebooks, c, head.grad_scale),
                             expected_losses, expected_grad)
        assert oracle.relative_error(expected_losses, gpu.download(losses)) < TOLERANCE, f"codebook {c}"
    assert oracle.relative_error(expected_grad, gpu.download(grad)) < TOLERANCE


def test_shape_checks_raise_the_reference_panics(gpu):
    logits, grad = gpu.zeros(Shape(4, 10)), gpu.zeros(Shape(4, 10))
    T = gpu.upload_tokens(np.zeros(8, np.uint32))
    with pytest.raises(AssertionError, match="cross_entropy: gradient shape"):
        gpu.cross_entropy(logits, T, CrossEntropyHead(0, 5, 2, 0, 1.0), gpu.zeros(Shape.vector(4)),
                          gpu.zeros(Shape(4, 9)))
    with pytest.raises(AssertionError, match="cross_entropy: head exceeds logits"):
        gpu.cross_entropy(logits, T, CrossEntropyHead(6, 5, 2, 0, 1.0), gpu.zeros(Shape.vector(4)), grad)
    with pytest.raises(AssertionError, match="cross_entropy: losses too small"):
        gpu.cross_entropy(logits, T, CrossEntropyHead(0, 5, 2, 0, 1.0), gpu.zeros(Shape.vector(3)), grad)
    with pytest.raises(AssertionError, match="cross_entropy: too few targets"):
        gpu.cross_entropy(logits, T, CrossEntropyHead(0, 5, 3, 0, 1.0), gpu.zeros(Shape.vector(4)), grad)
    assert gpu.download_tokens(T).tolist() == [0] * 8
