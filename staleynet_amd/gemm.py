"""Python view of the gfx950 GEMM library, shaped like the reference's host API.

Mirrors ``staleynet-cuda``'s GEMM surface so that callers and tests read like
the reference's own:

* ``Storage``, ``BatchStrides``, ``WriteMode`` and ``MatmulSpec`` with its
  builders (``crates/staleynet-cuda/src/ops/matmul.rs:14-142``,
  ``ops/mod.rs:251-269``);
* ``MatmulKernel`` and its ``tolerance`` (``device.rs:38-67``);
* ``Gpu`` with ``zeros/upload/download/copy_from_host/fill_zero/synchronize``
  and ``matmul`` (``device.rs:129-208``, ``ops/matmul.rs:144-171``);
* ``Shape`` and ``Tensor`` (``device.rs:210-275``).

Every call goes through the C ABI in ``include/staleynet_gemm.h``
(``libstaleynet_gemm.so``, built by ``staleynet_amd/build.py``). There is no
fallback: if the library is missing, loading raises.

Errors: the reference panics on undersized operands with
"matmul: left operand too small" etc.; here ``matmul`` raises
``MatmulPanic`` (an ``AssertionError``) with the same messages. Runtime
failures raise ``GpuError`` carrying the HIP status.
"""
from __future__ import annotations

import ctypes
import enum
import os
from dataclasses import dataclass, field, replace

import numpy as np

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
LIBRARY_PATH = os.path.join(PACKAGE_DIR, "libstaleynet_gemm.so")

# Status codes (include/staleynet_gemm.h).
SN_OK = 0
SN_ERR_NULL_ARGUMENT = -1
SN_ERR_LEFT_TOO_SMALL = -2
SN_ERR_RIGHT_TOO_SMALL = -3
SN_ERR_OUTPUT_TOO_SMALL = -4
SN_ERR_EMPTY_BATCH = -5
SN_ERR_OVERFLOW = -6
SN_ERR_UNSUPPORTED = -7
SN_ERR_ALIASING = -8
SN_ERR_NO_DEVICE = -9
SN_ERR_WORKSPACE = -10
SN_ERR_LENGTH_MISMATCH = -11
SN_ERR_SHAPE = -12

_VALIDATION_CODES = {SN_ERR_LEFT_TOO_SMALL, SN_ERR_RIGHT_TOO_SMALL, SN_ERR_OUTPUT_TOO_SMALL, SN_ERR_EMPTY_BATCH,
                     SN_ERR_OVERFLOW, SN_ERR_UNSUPPORTED, SN_ERR_ALIASING, SN_ERR_NULL_ARGUMENT,
                     SN_ERR_LENGTH_MISMATCH}


class Storage(enum.IntEnum):
    """How an operand is laid out relative to the logical matrix (ops/matmul.rs:15-22)."""

    RowMajor = 0
    Transposed = 1


class WriteMode(enum.IntEnum):
    """Overwrite or add into the output (ops/mod.rs:253-260); the value is the kernel flag."""

    Overwrite = 0
    Accumulate = 1


class Mask(enum.IntEnum):
    """Causal masks (an extension; ``None_`` is the reference's dense product)."""

    None_ = 0
    CausalOutput = 1
    CausalLeft = 2


class Precision(enum.IntEnum):
    """Per-call precision override (an extension)."""

    Default = 0
    F32 = 1
    Bf16 = 2


class MatmulKernel(enum.IntEnum):
    """Which GEMM implementation ``Gpu.matmul`` uses (the role of device.rs:38-54)."""

    MfmaF32 = 0
    MfmaBf16 = 1
    Simple = 2

    def tolerance(self) -> float:
        """Largest relative error the kernel's arithmetic allows (device.rs:56-66)."""
        return float(_library().sn_kernel_tolerance(int(self)))


@dataclass(frozen=True)
class BatchStrides:
    """Element offsets between consecutive matrices of a batch (ops/matmul.rs:35-54)."""

    count: int
    left: int
    right: int
    output: int


BatchStrides.SINGLE = BatchStrides(count=1, left=0, right=0, output=0)


@dataclass(frozen=True)
class MatmulSpec:
    """Full description of one (batched) GEMM (ops/matmul.rs:56-142)."""

    rows: int
    cols: int
    inner: int
    left: Storage = Storage.RowMajor
    right: Storage = Storage.RowMajor
    batch: BatchStrides = field(default_factory=lambda: BatchStrides.SINGLE)
    scale: float = 1.0
    write: WriteMode = WriteMode.Overwrite
    mask: Mask = Mask.None_
    query_offset: int = 0
    precision: Precision = Precision.Default

    @staticmethod
    def new(rows: int, cols: int, inner: int) -> "MatmulSpec":
        """``[rows, inner] · [inner, cols]``, row-major, unbatched, overwrite, scale 1."""
        return MatmulSpec(rows, cols, inner)

    def left_transposed(self) -> "MatmulSpec":
        return replace(self, left=Storage.Transposed)

    def right_transposed(self) -> "MatmulSpec":
        return replace(self, right=Storage.Transposed)

    def accumulate(self) -> "MatmulSpec":
        return replace(self, write=WriteMode.Accumulate)

    def scaled(self, scale: float) -> "MatmulSpec":
        return replace(self, scale=scale)

    def batched(self, strides: BatchStrides) -> "MatmulSpec":
        return replace(self, batch=strides)

    def causal_output(self, query_offset: int = 0) -> "MatmulSpec":
        """Outputs (q, k) with k > q + query_offset are not computed (written 0 / left unchanged)."""
        return replace(self, mask=Mask.CausalOutput, query_offset=query_offset)

    def causal_left(self, query_offset: int = 0) -> "MatmulSpec":
        """The stored left [query, key] matrix is 0 where k > q + query_offset."""
        return replace(self, mask=Mask.CausalLeft, query_offset=query_offset)

    def with_precision(self, precision: Precision) -> "MatmulSpec":
        return replace(self, precision=precision)

    def required_len(self, stride: int, per_matrix: int) -> int:
        """Elements an operand of ``per_matrix`` elements must hold (ops/matmul.rs:139-141)."""
        return (self.batch.count - 1) * stride + per_matrix

    def lengths(self) -> tuple[int, int, int]:
        """Elements the left, right and output buffers must hold."""
        return (self.required_len(self.batch.left, self.rows * self.inner),
                self.required_len(self.batch.right, self.inner * self.cols),
                self.required_len(self.batch.output, self.rows * self.cols))

    def flops(self) -> int:
        """Algorithmic floating-point operations, ``2·rows·cols·inner`` per matrix."""
        return 2 * self.rows * self.cols * self.inner * self.batch.count

    def to_c(self) -> "CMatmulSpec":
        return CMatmulSpec(self.rows, self.cols, self.inner, int(self.left), int(self.right), self.batch.count,
                           self.batch.left, self.batch.right, self.batch.output, float(self.scale), int(self.write),
                           int(self.mask), int(self.precision), self.query_offset)


class CMatmulSpec(ctypes.Structure):
    """``sn_matmul_spec`` (include/staleynet_gemm.h)."""

    _fields_ = [("rows", ctypes.c_size_t), ("cols", ctypes.c_size_t), ("inner", ctypes.c_size_t),
                ("left_storage", ctypes.c_uint32), ("right_storage", ctypes.c_uint32),
                ("batch_count", ctypes.c_size_t), ("batch_left", ctypes.c_size_t),
                ("batch_right", ctypes.c_size_t), ("batch_output", ctypes.c_size_t),
                ("scale", ctypes.c_float), ("write", ctypes.c_uint32), ("mask", ctypes.c_uint32),
                ("precision", ctypes.c_uint32), ("query_offset", ctypes.c_size_t)]


EMPTY_TOKEN = 0xFFFFFFFF  # crates/staleynet-cuda/src/kernels/mod.rs:46


@dataclass(frozen=True)
class CrossEntropyHead:
    """``CrossEntropyHead`` (crates/staleynet-cuda/src/ops/loss.rs:14-30)."""

    column_offset: int
    classes: int
    target_stride: int
    target_offset: int
    grad_scale: float


class CCrossEntropyHead(ctypes.Structure):
    _fields_ = [("column_offset", ctypes.c_size_t), ("classes", ctypes.c_size_t),
                ("target_stride", ctypes.c_size_t), ("target_offset", ctypes.c_size_t),
                ("grad_scale", ctypes.c_float)]


class CLaunchPlan(ctypes.Structure):
    """``sn_launch_plan``: how one product is launched (the role of launch.rs:28-48)."""
    _fields_ = [("path", ctypes.c_uint32), ("threads", ctypes.c_uint32), ("tile_rows", ctypes.c_uint32),
                ("tile_cols", ctypes.c_uint32), ("tiles_m", ctypes.c_uint32), ("tiles_n", ctypes.c_uint32),
                ("splits", ctypes.c_uint32), ("persistent_grid", ctypes.c_uint32), ("k_per_split", ctypes.c_uint64),
                ("batches_per_launch", ctypes.c_uint64), ("workgroups", ctypes.c_uint64),
                ("launches", ctypes.c_uint64), ("workspace_bytes", ctypes.c_uint64)]


# sn_launch_plan.path values (include/staleynet_gemm.h).
PATH_NONE, PATH_REFERENCE_ORDER, PATH_FEW_ROWS, PATH_FEW_ROWS_NT = 0, 1, 2, 3
PATH_F32_DIRECT, PATH_F32_REGISTER, PATH_BF16_STAGED, PATH_BF16_DIRECT, PATH_BF16_REGISTER = 4, 5, 6, 7, 8
PATH_BF16_WIDE, PATH_F32_DIRECT_SUMS, PATH_BF16_WIDE_SUMS, PATH_F32_PERSISTENT = 9, 10, 11, 12
TILED_PATHS = (PATH_F32_DIRECT, PATH_F32_REGISTER, PATH_BF16_STAGED, PATH_BF16_DIRECT, PATH_BF16_REGISTER,
               PATH_BF16_WIDE, PATH_F32_DIRECT_SUMS, PATH_BF16_WIDE_SUMS, PATH_F32_PERSISTENT)


class CAttentionShape(ctypes.Structure):
    _fields_ = [("heads", ctypes.c_size_t), ("queries", ctypes.c_size_t), ("keys", ctypes.c_size_t),
                ("head_dim", ctypes.c_size_t), ("q_stride", ctypes.c_size_t), ("kv_stride", ctypes.c_size_t),
                ("query_offset", ctypes.c_size_t), ("scale", ctypes.c_float)]


@dataclass(frozen=True)
class HeadLayout:
    """``HeadLayout`` (crates/staleynet-cuda/src/kernels/attention.rs:19-75)."""

    batch: int
    time: int
    heads: int
    head_dim: int
    width: int
    column_offset: int
    time_capacity: int
    time_offset: int

    @staticmethod
    def dense(batch: int, time: int, heads: int, head_dim: int, width: int, column_offset: int) -> "HeadLayout":
        return HeadLayout(batch, time, heads, head_dim, width, column_offset, time, 0)

    def in_cache(self, capacity: int, offset: int) -> "HeadLayout":
        return replace(self, time_capacity=capacity, time_offset=offset)

    def to_c(self) -> "CHeadLayout":
        return CHeadLayout(self.batch, self.time, self.heads, self.head_dim, self.width, self.column_offset,
                           self.time_capacity, self.time_offset)


class CHeadLayout(ctypes.Structure):
    _fields_ = [(name, ctypes.c_size_t) for name in ("batch", "time", "heads", "head_dim", "width", "column_offset",
                                                     "time_capacity", "time_offset")]


class TokenBuffer:
    """Token ids (u32) in device memory (``TokenBuffer``, device.rs:35-36)."""

    def __init__(self, gpu: "Gpu", pointer: int, count: int):
        self._gpu = gpu
        self.pointer = pointer
        self._count = count

    def __len__(self) -> int:
        return self._count

    def free(self) -> None:
        if self.pointer and self._gpu._ctx:  # as Tensor.free: a closed Gpu has no context to free through
            self._gpu._check(_library().sn_free_tokens(self._gpu._ctx, ctypes.c_void_p(self.pointer)), "free_tokens")
        self.pointer = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class GpuError(RuntimeError):
    """A failed call into the library; ``status`` is the C status code."""

    def __init__(self, status: int, what: str = ""):
        self.status = status
        super().__init__(f"{what + ': ' if what else ''}{status_string(status)} (status {status})")


class MatmulPanic(AssertionError):
    """The reference's ``assert!`` panics in ``Gpu::matmul`` (ops/matmul.rs:147-149)."""

    def __init__(self, status: int):
        self.status = status
        super().__init__(status_string(status))


_lib = None
_F32P = ctypes.POINTER(ctypes.c_float)


def _library() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIBRARY_PATH):
            raise FileNotFoundError(
                f"{LIBRARY_PATH} is missing; build it with `python -c 'import __graft_entry__ as g; g.build()'`")
        lib = ctypes.CDLL(LIBRARY_PATH)
        ctx = ctypes.c_void_p
        size = ctypes.c_size_t
        lib.sn_matmul_spec_new.argtypes = [size, size, size]
        lib.sn_matmul_spec_new.restype = CMatmulSpec
        lib.sn_context_create.argtypes = [ctypes.c_int, ctypes.POINTER(ctx)]
        lib.sn_context_create_with_workspace.argtypes = [ctypes.c_int, size, ctypes.POINTER(ctx)]
        lib.sn_context_destroy.argtypes = [ctx]
        lib.sn_context_bind.argtypes = [ctx]
        lib.sn_context_set_kernel.argtypes = [ctx, ctypes.c_uint32]
        lib.sn_context_get_kernel.argtypes = [ctx, ctypes.POINTER(ctypes.c_uint32)]
        lib.sn_context_stream.argtypes = [ctx]
        lib.sn_context_stream.restype = ctypes.c_void_p
        lib.sn_kernel_tolerance.argtypes = [ctypes.c_uint32]
        lib.sn_kernel_tolerance.restype = ctypes.c_float
        lib.sn_synchronize.argtypes = [ctx]
        lib.sn_alloc_zeroed.argtypes = [ctx, size, ctypes.POINTER(_F32P)]
        lib.sn_free.argtypes = [ctx, ctypes.c_void_p]
        lib.sn_upload.argtypes = [ctx, _F32P, size, ctypes.POINTER(_F32P)]
        lib.sn_download.argtypes = [ctx, ctypes.c_void_p, size, _F32P]
        lib.sn_copy_from_host.argtypes = [ctx, ctypes.c_void_p, _F32P, size]
        lib.sn_fill_zero.argtypes = [ctx, ctypes.c_void_p, size]
        lib.sn_matmul_validate.argtypes = [ctypes.POINTER(CMatmulSpec), size, size, size]
        lib.sn_matmul.argtypes = [ctx, ctypes.POINTER(CMatmulSpec), ctypes.c_void_p, size, ctypes.c_void_p, size,
                                  ctypes.c_void_p, size]
        lib.sn_status_string.argtypes = [ctypes.c_int]
        lib.sn_status_string.restype = ctypes.c_char_p
        lib.sn_fill_normal.argtypes = [ctypes.c_void_p, ctypes.c_void_p, size, ctypes.c_uint64, ctypes.c_uint64,
                                       ctypes.c_float, ctypes.c_float]
        lib.sn_copy_device.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, size]
        lib.sn_read_sum.argtypes = [ctypes.c_void_p, ctypes.c_void_p, size, ctypes.c_void_p, size]
        lib.sn_add_row_bias.argtypes = [ctx, ctypes.c_void_p, size, size, ctypes.c_void_p, size]
        lib.sn_accumulate_column_sums.argtypes = [ctx, ctypes.c_void_p, size, size, ctypes.c_void_p, size]
        lib.sn_matmul_bias.argtypes = [ctx, ctypes.POINTER(CMatmulSpec), ctypes.c_void_p, size, ctypes.c_void_p,
                                       size, ctypes.c_void_p, size, ctypes.c_void_p, size]
        lib.sn_matmul_column_sums.argtypes = [ctx, ctypes.POINTER(CMatmulSpec), ctypes.c_void_p, size,
                                              ctypes.c_void_p, size, ctypes.c_void_p, size, ctypes.c_void_p, size]
        lib.sn_causal_softmax.argtypes = [ctx, ctypes.c_void_p, size, size, size, ctypes.c_float, size]
        lib.sn_causal_attention.argtypes = [ctx, ctypes.POINTER(CAttentionShape), ctypes.c_void_p, size,
                                            ctypes.c_void_p, size, ctypes.c_void_p, size, ctypes.c_void_p, size,
                                            ctypes.c_void_p, size]
        lib.sn_causal_attention_score_grad.argtypes = [ctx, ctypes.POINTER(CAttentionShape), ctypes.c_void_p, size,
                                                       ctypes.c_void_p, size, ctypes.c_void_p, size,
                                                       ctypes.c_void_p, size, ctypes.c_void_p, size,
                                                       ctypes.c_void_p, size, ctypes.c_void_p, size]
        lib.sn_cross_entropy.argtypes = [ctx, ctypes.c_void_p, size, size, ctypes.c_void_p, size,
                                         ctypes.POINTER(CCrossEntropyHead), ctypes.c_void_p, size, ctypes.c_void_p,
                                         size, size]
        lib.sn_upload_tokens.argtypes = [ctx, ctypes.POINTER(ctypes.c_uint32), size,
                                         ctypes.POINTER(ctypes.c_void_p)]
        lib.sn_download_tokens.argtypes = [ctx, ctypes.c_void_p, size, ctypes.POINTER(ctypes.c_uint32)]
        lib.sn_free_tokens.argtypes = [ctx, ctypes.c_void_p]
        lib.sn_split_heads.argtypes = [ctx, ctypes.c_void_p, size, ctypes.c_void_p, size,
                                       ctypes.POINTER(CHeadLayout)]
        lib.sn_merge_heads.argtypes = [ctx, ctypes.c_void_p, size, ctypes.c_void_p, size,
                                       ctypes.POINTER(CHeadLayout)]
        lib.sn_softmax_backward.argtypes = [ctx, ctypes.c_void_p, size, size, ctypes.c_void_p, size, size]
        lib.sn_causal_attention_with_stats.argtypes = [ctx, ctypes.POINTER(CAttentionShape)] + \
            [ctypes.c_void_p, size] * 5
        lib.sn_causal_attention_backward.argtypes = [ctx, ctypes.POINTER(CAttentionShape)] + [ctypes.c_void_p, size] * 9
        lib.sn_plan_matmul.argtypes = [ctypes.POINTER(CMatmulSpec), ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p,
                                       ctypes.c_void_p, ctypes.c_uint32, size, ctypes.POINTER(CLaunchPlan)]
        lib.sn_plan_matmul_column_sums.argtypes = lib.sn_plan_matmul.argtypes
        lib.sn_matmul_noalloc.argtypes = [ctypes.POINTER(CMatmulSpec), ctypes.c_void_p, size, ctypes.c_void_p, size,
                                          ctypes.c_void_p, size, ctypes.c_void_p]
        u32p = ctypes.POINTER(ctypes.c_uint32)
        lib.sn_tile_map.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, u32p, u32p,
                                    u32p, u32p]
        for name in ("sn_context_create", "sn_context_create_with_workspace", "sn_context_destroy",
                     "sn_context_bind", "sn_context_set_kernel", "sn_context_get_kernel", "sn_synchronize",
                     "sn_alloc_zeroed", "sn_free", "sn_upload", "sn_download", "sn_copy_from_host", "sn_fill_zero",
                     "sn_matmul_validate", "sn_matmul", "sn_fill_normal", "sn_copy_device", "sn_read_sum",
                     "sn_add_row_bias", "sn_accumulate_column_sums", "sn_matmul_bias", "sn_causal_softmax",
                     "sn_softmax_backward", "sn_cross_entropy", "sn_upload_tokens", "sn_download_tokens",
                     "sn_free_tokens", "sn_split_heads", "sn_merge_heads", "sn_causal_attention",
                     "sn_causal_attention_score_grad", "sn_plan_matmul", "sn_plan_matmul_column_sums", "sn_matmul_column_sums", "sn_tile_map", "sn_matmul_noalloc", "sn_causal_attention_with_stats",
                     "sn_causal_attention_backward"):
            getattr(lib, name).restype = ctypes.c_int
        _lib = lib
    return _lib


def library() -> ctypes.CDLL:
    """The loaded ``libstaleynet_gemm.so`` (raises if it has not been built)."""
    return _library()


def status_string(status: int) -> str:
    return _library().sn_status_string(int(status)).decode()


def validate(spec: MatmulSpec, left_len: int, right_len: int, output_len: int) -> int:
    """``sn_matmul_validate``: the host checks of ``Gpu::matmul`` as a pure function."""
    c = spec.to_c()
    return int(_library().sn_matmul_validate(ctypes.byref(c), left_len, right_len, output_len))


# A device allocation's alignment (2 MiB): operands at such addresses take the aligned paths.
ALIGNED_ADDRESS = 1 << 40


def plan(spec: MatmulSpec, kernel: int = 0, cu_count: int = 256, workspace_bytes: int = 1536 << 20,
         left: int = ALIGNED_ADDRESS, right: int = 2 * ALIGNED_ADDRESS, output: int = 3 * ALIGNED_ADDRESS) -> CLaunchPlan:
    """``sn_plan_matmul``: the launch ``Gpu::matmul`` would make for ``spec`` (host only; the operand
    addresses are only inspected for alignment). Raises GpuError on a rejected spec."""
    c = spec.to_c()
    out = CLaunchPlan()
    rc = _library().sn_plan_matmul(ctypes.byref(c), kernel, left, right, output, cu_count, workspace_bytes,
                                   ctypes.byref(out))
    if rc != SN_OK:
        raise GpuError(rc, "plan_matmul")
    return out


def plan_column_sums(spec: MatmulSpec, kernel: int = 0, cu_count: int = 256, workspace_bytes: int = 1536 << 20,
                     left: int = ALIGNED_ADDRESS, right: int = 2 * ALIGNED_ADDRESS,
                     output: int = 3 * ALIGNED_ADDRESS) -> CLaunchPlan:
    """``sn_plan_matmul_column_sums``: the launch ``Gpu.matmul_column_sums`` would make (host only);
    path ``PATH_F32_DIRECT_SUMS`` or ``PATH_BF16_WIDE_SUMS`` when the column sums ride in the product's
    kernel."""
    c = spec.to_c()
    out = CLaunchPlan()
    rc = _library().sn_plan_matmul_column_sums(ctypes.byref(c), kernel, left, right, output, cu_count,
                                               workspace_bytes, ctypes.byref(out))
    if rc != SN_OK:
        raise GpuError(rc, "plan_matmul_column_sums")
    return out


def tile_map(workgroups: int, tiles_m: int, tiles_n: int, splits: int):
    """``sn_tile_map``: (matrix, slice, tile row, tile column) of each workgroup of a tiled launch,
    as four uint32 arrays."""
    arrays = [np.zeros(workgroups, np.uint32) for _ in range(4)]
    pointers = [a.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)) for a in arrays]
    rc = _library().sn_tile_map(workgroups, tiles_m, tiles_n, splits, *pointers)
    if rc != SN_OK:
        raise GpuError(rc, "tile_map")
    return tuple(arrays)


@dataclass(frozen=True)
class Shape:
    """Rows × columns of a row-major matrix (device.rs:210-243)."""

    rows: int
    cols: int

    @staticmethod
    def new(rows: int, cols: int) -> "Shape":
        return Shape(rows, cols)

    @staticmethod
    def vector(cols: int) -> "Shape":
        return Shape(1, cols)

    def __len__(self) -> int:
        return self.rows * self.cols


class Tensor:
    """A row-major f32 matrix in device memory owned by a ``Gpu`` (device.rs:245-275)."""

    def __init__(self, gpu: "Gpu", pointer: int, shape: Shape):
        self._gpu = gpu
        self.pointer = pointer
        self._shape = shape

    def shape(self) -> Shape:
        return self._shape

    def __len__(self) -> int:
        return len(self._shape)

    def reshaped(self, shape: Shape) -> "Tensor":
        assert len(shape) == len(self._shape), f"reshape {self._shape} -> {shape} changes size"
        out = Tensor(self._gpu, self.pointer, shape)
        self.pointer = 0  # ownership moves, as in the reference
        return out

    def free(self) -> None:
        if self.pointer and self._gpu._ctx:
            self._gpu._check(_library().sn_free(self._gpu._ctx, ctypes.c_void_p(self.pointer)), "free")
        self.pointer = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Gpu:
    """One device, one stream (``Gpu::new``, device.rs:147-155)."""

    def __init__(self, ordinal: int = 0, workspace_bytes: int | None = None):
        lib = _library()
        handle = ctypes.c_void_p()
        if workspace_bytes is None:
            rc = lib.sn_context_create(ordinal, ctypes.byref(handle))
        else:
            rc = lib.sn_context_create_with_workspace(ordinal, workspace_bytes, ctypes.byref(handle))
        if rc != SN_OK:
            raise GpuError(rc, f"Gpu::new({ordinal})")
        self._ctx = handle

    @staticmethod
    def new(ordinal: int = 0) -> "Gpu":
        return Gpu(ordinal)

    def close(self) -> None:
        if self._ctx:
            rc = _library().sn_context_destroy(self._ctx)
            self._ctx = None
            if rc != SN_OK:
                raise GpuError(rc, "destroy")

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc: int, what: str) -> None:
        if rc != SN_OK:
            raise GpuError(rc, what)

    @property
    def matmul_kernel(self) -> MatmulKernel:
        value = ctypes.c_uint32()
        self._check(_library().sn_context_get_kernel(self._ctx, ctypes.byref(value)), "get kernel")
        return MatmulKernel(value.value)

    @matmul_kernel.setter
    def matmul_kernel(self, kernel: MatmulKernel) -> None:
        self._check(_library().sn_context_set_kernel(self._ctx, int(kernel)), "set kernel")

    @property
    def stream(self) -> int:
        """The context's ``hipStream_t`` as an integer handle."""
        return int(_library().sn_context_stream(self._ctx) or 0)

    def bind_to_current_thread(self) -> None:
        self._check(_library().sn_context_bind(self._ctx), "bind")

    def synchronize(self) -> None:
        self._check(_library().sn_synchronize(self._ctx), "synchronize")

    def zeros(self, shape: Shape) -> Tensor:
        out = _F32P()
        self._check(_library().sn_alloc_zeroed(self._ctx, len(shape), ctypes.byref(out)), "zeros")
        return Tensor(self, ctypes.cast(out, ctypes.c_void_p).value or 0, shape)

    def upload(self, shape: Shape, values) -> Tensor:
        host = np.ascontiguousarray(values, dtype=np.float32).ravel()
        assert host.size == len(shape), f"upload: {host.size} values for shape {shape}"
        out = _F32P()
        self._check(_library().sn_upload(self._ctx, host.ctypes.data_as(_F32P), host.size, ctypes.byref(out)),
                    "upload")
        return Tensor(self, ctypes.cast(out, ctypes.c_void_p).value or 0, shape)

    def download(self, tensor: Tensor) -> np.ndarray:
        host = np.empty(len(tensor), np.float32)
        self._check(_library().sn_download(self._ctx, ctypes.c_void_p(tensor.pointer), host.size,
                                           host.ctypes.data_as(_F32P)), "download")
        return host

    def copy_from_host(self, tensor: Tensor, values) -> None:
        host = np.ascontiguousarray(values, dtype=np.float32).ravel()
        assert host.size == len(tensor)
        self._check(_library().sn_copy_from_host(self._ctx, ctypes.c_void_p(tensor.pointer),
                                                 host.ctypes.data_as(_F32P), host.size), "copy_from_host")

    def fill_zero(self, tensor: Tensor) -> None:
        self._check(_library().sn_fill_zero(self._ctx, ctypes.c_void_p(tensor.pointer), len(tensor)), "fill_zero")

    def fill_normal(self, tensor: Tensor, seed: int, stream_id: int, mean: float = 0.0, std: float = 1.0) -> None:
        """Seeded N(mean, std²) values (include/staleynet_synth.h), enqueued on this context's stream."""
        rc = _library().sn_fill_normal(ctypes.c_void_p(self.stream), ctypes.c_void_p(tensor.pointer), len(tensor),
                                       seed, stream_id, mean, std)
        self._check(rc, "fill_normal")

    def copy_device(self, dst: Tensor, src: Tensor) -> None:
        """Device-to-device copy by a plain streaming kernel (include/staleynet_synth.h), on this stream."""
        assert len(dst) == len(src), f"copy_device: {len(src)} values into {len(dst)}"
        rc = _library().sn_copy_device(ctypes.c_void_p(self.stream), ctypes.c_void_p(dst.pointer),
                                       ctypes.c_void_p(src.pointer), len(src))
        self._check(rc, "copy_device")

    def read_sum(self, src: Tensor, sums: Tensor) -> None:
        """Streaming read of ``src`` by ``len(sums)`` workgroups, each writing its share's sum
        (include/staleynet_synth.h): the practical HBM read-bandwidth probe."""
        rc = _library().sn_read_sum(ctypes.c_void_p(self.stream), ctypes.c_void_p(src.pointer), len(src),
                                    ctypes.c_void_p(sums.pointer), len(sums))
        self._check(rc, "read_sum")

    def matmul(self, spec: MatmulSpec, left: Tensor, right: Tensor, output: Tensor) -> None:
        """``Gpu::matmul``: enqueue ``output = scale·op(left)·op(right) (+ output)``."""
        self.matmul_raw(spec, left.pointer, len(left), right.pointer, len(right), output.pointer, len(output))

    def matmul_bias(self, spec: MatmulSpec, left: Tensor, right: Tensor, bias: Tensor, output: Tensor) -> None:
        """``Linear::forward``'s ``matmul`` then ``add_row_bias`` (linear.rs:46-47) in one pass
        (``sn_matmul_bias``): the bias is added in the product's epilogue, rounded as the two calls round."""
        c = spec.to_c()
        rc = _library().sn_matmul_bias(self._ctx, ctypes.byref(c), ctypes.c_void_p(left.pointer), len(left),
                                       ctypes.c_void_p(right.pointer), len(right), ctypes.c_void_p(bias.pointer),
                                       len(bias), ctypes.c_void_p(output.pointer), len(output))
        if rc in _VALIDATION_CODES:
            raise MatmulPanic(rc)
        self._check(rc, "matmul_bias")

    def matmul_column_sums(self, spec: MatmulSpec, left: Tensor, right: Tensor, output: Tensor, sums: Tensor) -> None:
        """``Linear::backward``'s weight-gradient ``matmul`` then ``accumulate_column_sums`` of the same
        output gradient (linear.rs:54-59) in one call (``sn_matmul_column_sums``): the product as ``matmul``
        computes it and ``sums[c] += Σ_k right[k, c]``, the sums taken inside the product where the fp32
        direct-to-LDS kernel or the bf16 256 x 256 kernel serves it."""
        c = spec.to_c()
        rc = _library().sn_matmul_column_sums(self._ctx, ctypes.byref(c), ctypes.c_void_p(left.pointer), len(left),
                                              ctypes.c_void_p(right.pointer), len(right),
                                              ctypes.c_void_p(output.pointer), len(output),
                                              ctypes.c_void_p(sums.pointer), len(sums))
        if rc in _VALIDATION_CODES:
            raise MatmulPanic(rc)
        self._check(rc, "matmul_column_sums")

    def add_row_bias(self, output: Tensor, bias: Tensor) -> None:
        """``Gpu::add_row_bias`` (ops/elementwise.rs:30-41): ``output[r, c] += bias[c]``."""
        rc = _library().sn_add_row_bias(self._ctx, ctypes.c_void_p(output.pointer), output.shape().rows,
                                        output.shape().cols, ctypes.c_void_p(bias.pointer), len(bias))
        if rc == SN_ERR_LENGTH_MISMATCH:
            raise AssertionError("add_row_bias: bias length must equal output columns")
        self._check(rc, "add_row_bias")

    def accumulate_column_sums(self, input: Tensor, sums: Tensor) -> None:
        """``Gpu::accumulate_column_sums`` (ops/elementwise.rs:43-58): ``sums += Σ_rows input``."""
        rc = _library().sn_accumulate_column_sums(self._ctx, ctypes.c_void_p(input.pointer), input.shape().rows,
                                                  input.shape().cols, ctypes.c_void_p(sums.pointer), len(sums))
        if rc == SN_ERR_LENGTH_MISMATCH:
            raise AssertionError("accumulate_column_sums: sums length must equal input columns")
        self._check(rc, "accumulate_column_sums")

    def causal_softmax(self, scores: Tensor, queries: int, scale: float, query_offset: int) -> None:
        """``Gpu::causal_softmax`` (ops/attention.rs:56-74), in place on ``[rows, keys]`` scores."""
        rc = _library().sn_causal_softmax(self._ctx, ctypes.c_void_p(scores.pointer), scores.shape().rows,
                                          scores.shape().cols, queries, scale, query_offset)
        if rc == SN_ERR_SHAPE:
            raise AssertionError("causal_softmax: rows must be a multiple of queries")
        self._check(rc, "causal_softmax")

    def causal_attention(self, q: Tensor, k: Tensor, v: Tensor, out: Tensor, heads: int, queries: int, keys: int,
                         head_dim: int, scale: float, query_offset: int = 0, q_stride: int | None = None,
                         kv_stride: int | None = None, probabilities: Tensor | None = None) -> None:
        """Fused causal attention forward (``sn_causal_attention``): ``out`` = O of the three calls of
        CausalSelfAttention::forward (layers/attention.rs:206-213) — scores, ``causal_softmax``, mix —
        and, when given, ``probabilities`` = the softmax they leave. Strides default to dense heads."""
        shape = CAttentionShape(heads, queries, keys, head_dim,
                                queries * head_dim if q_stride is None else q_stride,
                                keys * head_dim if kv_stride is None else kv_stride, query_offset, scale)
        p_pointer, p_len = (None, 0) if probabilities is None else (probabilities.pointer, len(probabilities))
        rc = _library().sn_causal_attention(self._ctx, ctypes.byref(shape), ctypes.c_void_p(q.pointer), len(q),
                                            ctypes.c_void_p(k.pointer), len(k), ctypes.c_void_p(v.pointer), len(v),
                                            ctypes.c_void_p(out.pointer), len(out), ctypes.c_void_p(p_pointer),
                                            p_len)
        if rc == SN_ERR_SHAPE:
            raise AssertionError("causal_attention: no keys")
        if rc == SN_ERR_LENGTH_MISMATCH:
            raise AssertionError("causal_attention: a buffer is too small for the shape")
        self._check(rc, "causal_attention")

    def causal_attention_score_grad(self, d_out: Tensor, v: Tensor, out: Tensor, probabilities: Tensor,
                                    grad: Tensor, heads: int, queries: int, keys: int, head_dim: int,
                                    query_offset: int = 0, q_stride: int | None = None,
                                    kv_stride: int | None = None, k: Tensor | None = None,
                                    q_grad: Tensor | None = None, scale: float = 1.0) -> None:
        """Fused probability gradient (``sn_causal_attention_score_grad``): ``grad`` = what the dP
        product and ``softmax_backward`` of CausalSelfAttention::backward (layers/attention.rs:238-248)
        leave in ``grads.probabilities``; with ``k`` and ``q_grad``, also the next call's
        ``grads.queries`` = scale * grad * K (:250-253)."""
        shape = CAttentionShape(heads, queries, keys, head_dim,
                                queries * head_dim if q_stride is None else q_stride,
                                keys * head_dim if kv_stride is None else kv_stride, query_offset, scale)
        k_pointer, k_len = (None, 0) if k is None else (k.pointer, len(k))
        q_pointer, q_len = (None, 0) if q_grad is None else (q_grad.pointer, len(q_grad))
        rc = _library().sn_causal_attention_score_grad(
            self._ctx, ctypes.byref(shape), ctypes.c_void_p(d_out.pointer), len(d_out), ctypes.c_void_p(v.pointer),
            len(v), ctypes.c_void_p(out.pointer), len(out), ctypes.c_void_p(probabilities.pointer),
            len(probabilities), ctypes.c_void_p(grad.pointer), len(grad), ctypes.c_void_p(k_pointer), k_len,
            ctypes.c_void_p(q_pointer), q_len)
        if rc == SN_ERR_SHAPE:
            raise AssertionError("causal_attention_score_grad: no keys")
        if rc == SN_ERR_LENGTH_MISMATCH:
            raise AssertionError("causal_attention_score_grad: a buffer is too small for the shape")
        self._check(rc, "causal_attention_score_grad")

    def causal_attention_with_stats(self, q: Tensor, k: Tensor, v: Tensor, out: Tensor, stats: Tensor, heads: int,
                                    queries: int, keys: int, head_dim: int, scale: float, query_offset: int = 0,
                                    q_stride: int | None = None, kv_stride: int | None = None) -> None:
        """Training forward without the probabilities (``sn_causal_attention_with_stats``): ``out`` = O as
        ``causal_attention`` gives it, ``stats`` = per query {m, l}, from which the backward rebuilds P."""
        shape = CAttentionShape(heads, queries, keys, head_dim,
                                queries * head_dim if q_stride is None else q_stride,
                                keys * head_dim if kv_stride is None else kv_stride, query_offset, scale)
        rc = _library().sn_causal_attention_with_stats(
            self._ctx, ctypes.byref(shape), ctypes.c_void_p(q.pointer), len(q), ctypes.c_void_p(k.pointer), len(k),
            ctypes.c_void_p(v.pointer), len(v), ctypes.c_void_p(out.pointer), len(out),
            ctypes.c_void_p(stats.pointer), len(stats))
        if rc == SN_ERR_SHAPE:
            raise AssertionError("causal_attention_with_stats: no keys")
        if rc == SN_ERR_LENGTH_MISMATCH:
            raise AssertionError("causal_attention_with_stats: a buffer is too small for the shape")
        self._check(rc, "causal_attention_with_stats")

    def causal_attention_backward(self, q: Tensor, k: Tensor, v: Tensor, out: Tensor, d_out: Tensor, stats: Tensor,
                                  q_grad: Tensor, k_grad: Tensor, v_grad: Tensor, heads: int, queries: int, keys: int,
                                  head_dim: int, scale: float, query_offset: int = 0, q_stride: int | None = None,
                                  kv_stride: int | None = None) -> None:
        """The attention backward from O and the statistics (``sn_causal_attention_backward``):
        ``q_grad``, ``k_grad``, ``v_grad`` = the grads.queries, grads.keys and grads.values that
        CausalSelfAttention::backward (layers/attention.rs:238-260) leaves, with no P or dS in memory."""
        shape = CAttentionShape(heads, queries, keys, head_dim,
                                queries * head_dim if q_stride is None else q_stride,
                                keys * head_dim if kv_stride is None else kv_stride, query_offset, scale)
        args = [self._ctx, ctypes.byref(shape)]
        for t in (q, k, v, out, d_out, stats, q_grad, k_grad, v_grad):
            args += [ctypes.c_void_p(t.pointer), len(t)]
        rc = _library().sn_causal_attention_backward(*args)
        if rc == SN_ERR_SHAPE:
            raise AssertionError("causal_attention_backward: no keys")
        if rc == SN_ERR_LENGTH_MISMATCH:
            raise AssertionError("causal_attention_backward: a buffer is too small for the shape")
        self._check(rc, "causal_attention_backward")

    def softmax_backward(self, probabilities: Tensor, grad: Tensor) -> None:
        """``Gpu::softmax_backward`` (ops/attention.rs:76-92), in place on ``grad``."""
        p, g = probabilities.shape(), grad.shape()
        rc = _library().sn_softmax_backward(self._ctx, ctypes.c_void_p(probabilities.pointer), p.rows, p.cols,
                                            ctypes.c_void_p(grad.pointer), g.rows, g.cols)
        if rc == SN_ERR_SHAPE:
            raise AssertionError("softmax_backward: shape mismatch")
        self._check(rc, "softmax_backward")

    def _permute_heads(self, fn, src: Tensor, dst: Tensor, layout: HeadLayout, packed: Tensor,
                       head_major: Tensor) -> None:
        assert layout.time_offset + layout.time <= layout.time_capacity, "HeadLayout: time range exceeds capacity"
        assert len(packed) >= layout.batch * layout.time * layout.width, "HeadLayout: packed tensor too small"
        assert len(head_major) >= layout.batch * layout.heads * layout.time_capacity * layout.head_dim, \
            "HeadLayout: head-major tensor too small"
        c = layout.to_c()
        self._check(fn(self._ctx, ctypes.c_void_p(src.pointer), len(src), ctypes.c_void_p(dst.pointer), len(dst),
                       ctypes.byref(c)), "permute heads")

    def split_heads(self, packed: Tensor, head_major: Tensor, layout: HeadLayout) -> None:
        """``Gpu::split_heads`` (ops/attention.rs:20-35): packed columns -> head-major."""
        self._permute_heads(_library().sn_split_heads, packed, head_major, layout, packed, head_major)

    def merge_heads(self, head_major: Tensor, packed: Tensor, layout: HeadLayout) -> None:
        """``Gpu::merge_heads`` (ops/attention.rs:37-52): head-major -> packed columns."""
        self._permute_heads(_library().sn_merge_heads, head_major, packed, layout, packed, head_major)

    def upload_tokens(self, tokens) -> TokenBuffer:
        """``Gpu::upload_tokens`` (device.rs:194-197)."""
        host = np.ascontiguousarray(tokens, dtype=np.uint32).ravel()
        out = ctypes.c_void_p()
        self._check(_library().sn_upload_tokens(self._ctx, host.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                                                host.size, ctypes.byref(out)), "upload_tokens")
        return TokenBuffer(self, out.value or 0, host.size)

    def download_tokens(self, tokens: TokenBuffer) -> np.ndarray:
        host = np.empty(len(tokens), np.uint32)
        self._check(_library().sn_download_tokens(self._ctx, ctypes.c_void_p(tokens.pointer), host.size,
                                                  host.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32))),
                    "download_tokens")
        return host

    def cross_entropy(self, logits: Tensor, targets: TokenBuffer, head: CrossEntropyHead, losses: Tensor,
                      logits_grad: Tensor) -> None:
        """``Gpu::cross_entropy`` (ops/loss.rs:34-71): losses and the head's columns of the gradient."""
        shape = logits.shape()
        assert logits_grad.shape() == shape, "cross_entropy: gradient shape"
        assert head.column_offset + head.classes <= shape.cols, "cross_entropy: head exceeds logits"
        assert len(losses) >= shape.rows, "cross_entropy: losses too small"
        assert len(targets) >= shape.rows * head.target_stride, "cross_entropy: too few targets"
        c = CCrossEntropyHead(head.column_offset, head.classes, head.target_stride, head.target_offset,
                              head.grad_scale)
        rc = _library().sn_cross_entropy(self._ctx, ctypes.c_void_p(logits.pointer), shape.rows, shape.cols,
                                         ctypes.c_void_p(targets.pointer), len(targets), ctypes.byref(c),
                                         ctypes.c_void_p(losses.pointer), len(losses),
                                         ctypes.c_void_p(logits_grad.pointer), logits_grad.shape().rows,
                                         logits_grad.shape().cols)
        self._check(rc, "cross_entropy")

    def matmul_raw(self, spec: MatmulSpec, left: int, left_len: int, right: int, right_len: int, output: int,
                   output_len: int) -> None:
        """``sn_matmul`` on raw device pointers (for buffers owned elsewhere)."""
        c = spec.to_c()
        rc = _library().sn_matmul(self._ctx, ctypes.byref(c), ctypes.c_void_p(left), left_len,
                                  ctypes.c_void_p(right), right_len, ctypes.c_void_p(output), output_len)
        if rc in _VALIDATION_CODES:
            raise MatmulPanic(rc)
        self._check(rc, "matmul")
