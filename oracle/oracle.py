"""ctypes view of the CPU oracle (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg import this module, and only to check or time against the GPU path; the
product library never routes through it. The arithmetic lives in
``oracle/matmul_oracle.c`` and follows the reference's CPU GEMM,
``crates/staleynet-cuda/src/reference.rs:10-38``.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(_HERE, "liboracle.so")

_size = ctypes.c_size_t
_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_lib = None


def load() -> ctypes.CDLL:
    """Loads ``liboracle.so`` (built by ``make -C oracle``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY_PATH):
            raise FileNotFoundError(f"{LIBRARY_PATH} is missing: run `make -C oracle` (or __graft_entry__.build())")
        lib = ctypes.CDLL(LIBRARY_PATH)
        common = [_size, _size, _size, ctypes.c_int, ctypes.c_int]
        lib.oracle_matmul.argtypes = common + [_size, _size, _size, _size, ctypes.c_float, ctypes.c_int,
                                               _f32p, _f32p, _f32p]
        lib.oracle_matmul.restype = None
        lib.oracle_matmul_rows.argtypes = common + [_size, _size, _size, _size, ctypes.c_float, ctypes.c_int,
                                                    _f32p, _f32p, _f32p, _size, _size]
        lib.oracle_matmul_rows.restype = None
        lib.oracle_matmul_elements.argtypes = common + [_size, _size, ctypes.c_float, ctypes.c_int, _f32p, _f32p,
                                                        _size, _u64p, _u64p, _u64p, _f32p, _f32p]
        lib.oracle_matmul_elements.restype = None
        lib.oracle_matmul_f64.argtypes = common + [_size, _size, ctypes.c_double, ctypes.c_int, _f32p, _f32p,
                                                   _size, _u64p, _u64p, _u64p, _f32p, _f64p]
        lib.oracle_matmul_f64.restype = None
        lib.oracle_random_values.argtypes = [_size, ctypes.c_uint64, _f32p]
        lib.oracle_random_values.restype = None
        lib.oracle_relative_error.argtypes = [_f32p, _f32p, _size]
        lib.oracle_relative_error.restype = ctypes.c_float
        lib.oracle_causal_softmax.argtypes = [_f32p, _size, _size, _size, ctypes.c_float, _size]
        lib.oracle_causal_softmax.restype = None
        lib.oracle_softmax_backward.argtypes = [_f32p, _f32p, _size, _size]
        lib.oracle_softmax_backward.restype = None
        lib.oracle_add_row_bias.argtypes = [_f32p, _size, _size, _f32p]
        lib.oracle_add_row_bias.restype = None
        lib.oracle_accumulate_column_sums.argtypes = [_f32p, _size, _size, _f32p, _f32p]
        lib.oracle_accumulate_column_sums.restype = None
        lib.oracle_column_sums_f64.argtypes = [_f32p, _size, _size, _f32p, _f64p]
        lib.oracle_column_sums_f64.restype = None
        lib.oracle_split_heads.argtypes = [_f32p, _f32p, ctypes.POINTER(_size)]
        lib.oracle_split_heads.restype = None
        lib.oracle_merge_heads.argtypes = [_f32p, _f32p, ctypes.POINTER(_size)]
        lib.oracle_merge_heads.restype = None
        lib.oracle_cross_entropy.argtypes = [_f32p, ctypes.POINTER(ctypes.c_uint32), _size, _size, _size, _size,
                                             _size, _size, ctypes.c_float, _f32p, _f32p]
        lib.oracle_cross_entropy.restype = None
        _lib = lib
    return _lib


def _f32(array: np.ndarray):
    assert array.dtype == np.float32 and array.flags["C_CONTIGUOUS"]
    return array.ctypes.data_as(_f32p)


def _u64(array: np.ndarray):
    assert array.dtype == np.uint64 and array.flags["C_CONTIGUOUS"]
    return array.ctypes.data_as(_u64p)


@dataclass(frozen=True)
class Product:
    """The fields of the reference's ``MatmulSpec`` (ops/matmul.rs:58-82) the oracle needs."""

    rows: int
    cols: int
    inner: int
    left_transposed: bool = False
    right_transposed: bool = False
    count: int = 1
    batch_left: int = 0
    batch_right: int = 0
    batch_output: int = 0
    scale: float = 1.0
    accumulate: bool = False

    def _head(self):
        return (self.rows, self.cols, self.inner, int(self.left_transposed), int(self.right_transposed))


def matmul(p: Product, left: np.ndarray, right: np.ndarray, output: np.ndarray) -> None:
    """``reference::matmul`` on host arrays; ``output`` is updated in place."""
    load().oracle_matmul(*p._head(), p.count, p.batch_left, p.batch_right, p.batch_output, p.scale,
                         int(p.accumulate), _f32(left), _f32(right), _f32(output))


def matmul_rows(p: Product, left, right, output, row_begin: int, row_end: int) -> None:
    """``reference::matmul`` restricted to rows ``[row_begin, row_end)`` of every matrix."""
    load().oracle_matmul_rows(*p._head(), p.count, p.batch_left, p.batch_right, p.batch_output, p.scale,
                              int(p.accumulate), _f32(left), _f32(right), _f32(output), row_begin, row_end)


def matmul_elements(p: Product, left, right, batch, row, col, previous=None) -> np.ndarray:
    """Reference-order values at the given (batch, row, col) positions."""
    batch, row, col = (np.ascontiguousarray(x, dtype=np.uint64) for x in (batch, row, col))
    n = batch.size
    prev = np.zeros(n, np.float32) if previous is None else np.ascontiguousarray(previous, np.float32)
    out = np.empty(n, np.float32)
    load().oracle_matmul_elements(*p._head(), p.batch_left, p.batch_right, p.scale, int(p.accumulate),
                                  _f32(left), _f32(right), n, _u64(batch), _u64(row), _u64(col), _f32(prev),
                                  _f32(out))
    return out


def matmul_elements_f64(p: Product, left, right, batch, row, col, previous=None) -> np.ndarray:
    """The same positions accumulated in f64 (an error yardstick, not the parity target)."""
    batch, row, col = (np.ascontiguousarray(x, dtype=np.uint64) for x in (batch, row, col))
    n = batch.size
    prev = np.zeros(n, np.float32) if previous is None else np.ascontiguousarray(previous, np.float32)
    out = np.empty(n, np.float64)
    load().oracle_matmul_f64(*p._head(), p.batch_left, p.batch_right, float(p.scale), int(p.accumulate),
                             _f32(left), _f32(right), n, _u64(batch), _u64(row), _u64(col), _f32(prev),
                             out.ctypes.data_as(_f64p))
    return out


def random_values(count: int, seed: int) -> np.ndarray:
    """The reference test's LCG values in [-1, 1) (kernels_match_reference.rs:26-38)."""
    out = np.empty(count, np.float32)
    load().oracle_random_values(count, seed, _f32(out))
    return out


def relative_error(expected: np.ndarray, actual: np.ndarray) -> float:
    """The reference test's metric (kernels_match_reference.rs:41-52)."""
    expected = np.ascontiguousarray(expected, np.float32).ravel()
    actual = np.ascontiguousarray(actual, np.float32).ravel()
    assert expected.size == actual.size
    return float(load().oracle_relative_error(_f32(expected), _f32(actual), expected.size))


def causal_softmax(scores: np.ndarray, queries: int, keys: int, scale: float, query_offset: int) -> None:
    """``reference::causal_softmax`` in place on ``[rows, keys]`` (reference.rs:101-119)."""
    assert scores.size % keys == 0
    load().oracle_causal_softmax(_f32(scores), scores.size // keys, queries, keys, scale, query_offset)


def softmax_backward(probabilities: np.ndarray, grad: np.ndarray, cols: int) -> None:
    """``reference::softmax_backward`` in place on ``grad`` (reference.rs:122-137)."""
    assert probabilities.size == grad.size and grad.size % cols == 0
    load().oracle_softmax_backward(_f32(probabilities), _f32(grad), grad.size // cols, cols)


def add_row_bias(output: np.ndarray, cols: int, bias: np.ndarray) -> None:
    """``output[r, c] += bias[c]`` in place on ``[rows, cols]`` (kernels/elementwise.rs:62-68)."""
    assert output.size % cols == 0 and bias.size == cols
    load().oracle_add_row_bias(_f32(output), output.size // cols, cols, _f32(bias))


def accumulate_column_sums(values: np.ndarray, cols: int, sums: np.ndarray) -> None:
    """``sums[c] += Σ_r values[r, c]``, each column summed in row order in f32
    (kernels/elementwise.rs:78-93); ``sums`` is updated in place."""
    assert values.size % cols == 0 and sums.size == cols
    scratch = np.empty(cols, np.float32)
    load().oracle_accumulate_column_sums(_f32(values), values.size // cols, cols, _f32(sums), _f32(scratch))


def column_sums_f64(values: np.ndarray, cols: int, initial: np.ndarray) -> np.ndarray:
    """``initial + Σ_r values[r, :]`` in f64 (an error yardstick, not the parity target)."""
    assert values.size % cols == 0 and initial.size == cols
    out = np.empty(cols, np.float64)
    load().oracle_column_sums_f64(_f32(values), values.size // cols, cols, _f32(initial), out.ctypes.data_as(_f64p))
    return out


@dataclass(frozen=True)
class HeadLayout:
    """``HeadLayout`` (crates/staleynet-cuda/src/kernels/attention.rs:19-43)."""

    batch: int
    time: int
    heads: int
    head_dim: int
    width: int
    column_offset: int
    time_capacity: int
    time_offset: int

    def _c(self):
        return (_size * 8)(self.batch, self.time, self.heads, self.head_dim, self.width, self.column_offset,
                           self.time_capacity, self.time_offset)


def split_heads(packed: np.ndarray, head_major: np.ndarray, layout: HeadLayout) -> None:
    """Packed columns -> head-major (kernels/attention.rs:113-121), in place on ``head_major``."""
    load().oracle_split_heads(_f32(packed), _f32(head_major), layout._c())


def merge_heads(head_major: np.ndarray, packed: np.ndarray, layout: HeadLayout) -> None:
    """Head-major -> packed columns (kernels/attention.rs:130-138), in place on ``packed``."""
    load().oracle_merge_heads(_f32(head_major), _f32(packed), layout._c())


EMPTY_TOKEN = 0xFFFFFFFF  # crates/staleynet-cuda/src/kernels/mod.rs:46


@dataclass(frozen=True)
class CrossEntropyHead:
    """``CrossEntropyHead`` (crates/staleynet-cuda/src/ops/loss.rs:14-30)."""

    column_offset: int
    classes: int
    target_stride: int
    target_offset: int
    grad_scale: float


def cross_entropy(logits: np.ndarray, targets: np.ndarray, cols: int, head: CrossEntropyHead,
                  losses: np.ndarray, grad: np.ndarray) -> None:
    """``reference::cross_entropy`` (reference.rs:139-166): ``losses`` and the head's columns of
    ``grad`` are written in place."""
    targets = np.ascontiguousarray(targets, np.uint32)
    rows = losses.size
    assert logits.size == grad.size == rows * cols and targets.size >= rows * head.target_stride
    load().oracle_cross_entropy(_f32(logits), targets.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), rows, cols,
                                head.column_offset, head.classes, head.target_stride, head.target_offset,
                                head.grad_scale, _f32(losses), _f32(grad))


def _workers(workers):
    return max(1, workers or min(16, os.cpu_count() or 1))


def matmul_parallel(p: Product, left, right, output, workers: int | None = None) -> None:
    """``matmul`` with output rows split across threads (ctypes releases the
    GIL); every element is computed exactly as in the serial loop."""
    from concurrent.futures import ThreadPoolExecutor

    n = _workers(workers)
    bounds = [p.rows * i // n for i in range(n + 1)]
    with ThreadPoolExecutor(n) as pool:
        list(pool.map(lambda i: matmul_rows(p, left, right, output, bounds[i], bounds[i + 1]), range(n)))


def matmul_elements_parallel(p: Product, left, right, batch, row, col, previous=None, workers=None, f64=False):
    """``matmul_elements`` (or its f64 twin) with the positions split across threads."""
    from concurrent.futures import ThreadPoolExecutor

    batch, row, col = (np.ascontiguousarray(x, dtype=np.uint64) for x in (batch, row, col))
    prev = None if previous is None else np.ascontiguousarray(previous, np.float32)
    n = _workers(workers)
    bounds = [batch.size * i // n for i in range(n + 1)]
    fn = matmul_elements_f64 if f64 else matmul_elements

    def part(i):
        s = slice(bounds[i], bounds[i + 1])
        return fn(p, left, right, batch[s], row[s], col[s], None if prev is None else prev[s])

    with ThreadPoolExecutor(n) as pool:
        return np.concatenate(list(pool.map(part, range(n))))
