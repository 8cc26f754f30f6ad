"""Benchmark of the GEMM hot path on one MI355X.

Workload (BASELINE.json metric, config 2): the 111.5M model's training GEMM
set, exactly as the reference's model issues it through ``Gpu::matmul``:
12 blocks x {QKV 768->2304, out-proj 768->768, FFN up 768->3072, FFN down
3072->768}, each as forward NN (``Linear::forward``, linear.rs:43-48),
input-gradient NT and weight-gradient TN with accumulate
(``Linear::backward``, linear.rs:51-63), plus the 16-codebook head
768->16384 (gpt.rs:72) in the same three forms; M = 16 x 2048 = 32768
tokens. 19.173 TFLOP of algorithmic work per step. Inputs are seeded
synthetic data resident in HBM before timing (activations and gradients
~N(0,1), weights ~N(0,0.02)).

A "step" is one pass over that set. The line printed is the driver's JSON
contract plus ``roofline`` (the forward NN kernel, timed per launch with HIP
events on the library's stream) and ``cpu_baseline`` (the reference's CPU
matmul restated bit-for-bit in oracle/, on one host core, over a bounded
row sample of every GEMM of the set, scaled to the full set).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from staleynet_amd.gemm import BatchStrides, Gpu, MatmulSpec, Shape  # noqa: E402

# MI355X published peaks (dense): fp32 matrix 157.3 TFLOP/s, bf16 2.5 PFLOP/s, HBM 8 TB/s.
PEAK_FP32_TFLOPS = 157.3
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
SEED = 1234


class HipEvents:
    """hipEvent timing on an explicit stream (the library's own)."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]

    def create(self) -> ctypes.c_void_p:
        event = ctypes.c_void_p()
        assert self.hip.hipEventCreate(ctypes.byref(event)) == 0
        return event

    def record(self, event, stream: int) -> None:
        assert self.hip.hipEventRecord(event, ctypes.c_void_p(stream)) == 0

    def elapsed_ms(self, start, end) -> float:
        ms = ctypes.c_float()
        assert self.hip.hipEventSynchronize(end) == 0
        assert self.hip.hipEventElapsedTime(ctypes.byref(ms), start, end) == 0
        return float(ms.value)

    def device_synchronize(self) -> None:
        assert self.hip.hipDeviceSynchronize() == 0

    def destroy(self, event) -> None:
        self.hip.hipEventDestroy(event)


# ---- the workload ---------------------------------------------------------------

MODEL_111M = dict(name="111.5M", blocks=12, width=768, ffn=3072, heads_width=16 * 1024, tokens=16 * 2048)


def linear_products(tokens: int, inputs: int, outputs: int):
    """The three products of one Linear (linear.rs:43-63): forward NN, dW TN (accumulate), dX NT."""
    return [
        ("NN", MatmulSpec.new(tokens, outputs, inputs)),
        ("TN", MatmulSpec.new(inputs, outputs, tokens).left_transposed().accumulate()),
        ("NT", MatmulSpec.new(tokens, inputs, outputs).right_transposed()),
    ]


def training_set(model=MODEL_111M):
    """(label, layout, spec, operands) for every GEMM of one training step's set."""
    m, d, f = model["tokens"], model["width"], model["ffn"]
    layers = [("qkv", d, 3 * d), ("out", d, d), ("up", d, f), ("down", f, d)]
    items = []
    for block in range(model["blocks"]):
        for name, inputs, outputs in layers:
            items.append((f"b{block}.{name}", inputs, outputs))
    items.append(("head", d, model["heads_width"]))
    return items


class LinearBuffers:
    """Device tensors of one Linear: x [M,in], w [in,out], dy [M,out], y, dx, dw."""

    def __init__(self, gpu: Gpu, tokens: int, inputs: int, outputs: int, stream_base: int):
        self.x = gpu.zeros(Shape(tokens, inputs))
        self.w = gpu.zeros(Shape(inputs, outputs))
        self.dy = gpu.zeros(Shape(tokens, outputs))
        self.y = gpu.zeros(Shape(tokens, outputs))
        self.dx = gpu.zeros(Shape(tokens, inputs))
        self.dw = gpu.zeros(Shape(inputs, outputs))
        gpu.fill_normal(self.x, SEED, stream_base + 0, 0.0, 1.0)
        gpu.fill_normal(self.w, SEED, stream_base + 1, 0.0, 0.02)
        gpu.fill_normal(self.dy, SEED, stream_base + 2, 0.0, 1.0)

    def operands(self, layout: str):
        if layout == "NN":
            return self.x, self.w, self.y
        if layout == "TN":
            return self.x, self.dy, self.dw
        return self.dy, self.w, self.dx


def build_set(gpu: Gpu, model=MODEL_111M):
    calls = []
    buffers = []
    for index, (label, inputs, outputs) in enumerate(training_set(model)):
        buf = LinearBuffers(gpu, model["tokens"], inputs, outputs, 16 * index)
        buffers.append(buf)
        for layout, spec in linear_products(model["tokens"], inputs, outputs):
            calls.append((label, layout, spec, buf.operands(layout)))
    gpu.synchronize()
    return calls, buffers


def run_step(gpu: Gpu, calls, events=None, marks=None, stream=0):
    for i, (_, _, spec, (left, right, out)) in enumerate(calls):
        if marks is not None:
            events.record(marks[i], stream)
        gpu.matmul(spec, left, right, out)
    if marks is not None:
        events.record(marks[len(calls)], stream)


# ---- CPU baseline -----------------------------------------------------------------

def cpu_baseline(gpu: Gpu, calls, budget_s: float):
    """Times the oracle (reference::matmul restated in C, one core) on a row
    sample of each distinct GEMM of the set, using the GPU's own input bytes,
    and scales each to its full size (cost is linear in output rows)."""
    from oracle import oracle

    distinct = {}
    for label, layout, spec, ops in calls:
        key = (layout, spec.rows, spec.cols, spec.inner)
        distinct.setdefault(key, [spec, ops, 0])
        distinct[key][2] += 1
    per_gemm_budget = budget_s / len(distinct)
    projected_s = 0.0
    sampled_flops = 0
    sampled_s = 0.0
    samples = []
    for (layout, rows, cols, inner), (spec, (left, right, out), count) in distinct.items():
        a = gpu.download(left)
        b = gpu.download(right)
        c = np.zeros(rows * cols, np.float32) if spec.write == 0 else gpu.download(out)
        product = oracle.Product(rows, cols, inner, bool(spec.left), bool(spec.right), 1, 0, 0, 0, spec.scale,
                                 bool(spec.write))
        # One row first to size the sample, then as many rows as fit the budget.
        t0 = time.perf_counter()
        oracle.matmul_rows(product, a, b, c, 0, 1)
        one_row = max(time.perf_counter() - t0, 1e-6)
        n_rows = int(max(1, min(rows - 1, per_gemm_budget / one_row)))
        t0 = time.perf_counter()
        oracle.matmul_rows(product, a, b, c, 1, 1 + n_rows)
        elapsed = time.perf_counter() - t0
        rate = 2.0 * n_rows * cols * inner / elapsed
        projected_s += count * spec.flops() / rate
        sampled_flops += 2 * n_rows * cols * inner
        sampled_s += elapsed
        samples.append(f"{layout} {rows}x{cols}x{inner}: {n_rows} rows")
        del a, b, c
    return projected_s, sampled_flops, sampled_s, samples


# ---- main --------------------------------------------------------------------------

def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=5)
    parser.add_argument("--warmup", type=int, default=1)
    parser.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU-baseline sampling")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = parser.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (the GEMM path has no multi-GPU component); got --gpus {args.gpus}",
              file=sys.stderr)
        return 2

    gpu = Gpu(0)
    events = HipEvents()
    stream = gpu.stream
    calls, _buffers = build_set(gpu)
    set_flops = sum(spec.flops() for _, _, spec, _ in calls)

    for _ in range(args.warmup):
        run_step(gpu, calls)
    events.device_synchronize()

    marks = [[events.create() for _ in range(len(calls) + 1)] for _ in range(args.steps)]
    start, end = events.create(), events.create()
    events.device_synchronize()
    events.record(start, stream)
    for step in range(args.steps):
        run_step(gpu, calls, events, marks[step], stream)
    events.record(end, stream)
    events.device_synchronize()
    total_ms = events.elapsed_ms(start, end)
    ms_per_step = total_ms / args.steps

    per_call_ms = np.zeros((args.steps, len(calls)))
    for step in range(args.steps):
        for i in range(len(calls)):
            per_call_ms[step, i] = events.elapsed_ms(marks[step][i], marks[step][i + 1])
    mean_ms = per_call_ms.mean(axis=0)

    layouts = {}
    for i, (label, layout, spec, _) in enumerate(calls):
        entry = layouts.setdefault(layout, {"flops": 0, "ms": 0.0, "launches": 0})
        entry["flops"] += spec.flops()
        entry["ms"] += mean_ms[i]
        entry["launches"] += 1
    per_layout = {k: {"tflops": v["flops"] / (v["ms"] * 1e-3) / 1e12, "ms_per_step": v["ms"],
                      "frac_fp32_peak": v["flops"] / (v["ms"] * 1e-3) / 1e12 / PEAK_FP32_TFLOPS}
                  for k, v in layouts.items()}
    shapes = {}
    for i, (label, layout, spec, _) in enumerate(calls):
        key = f"{layout} {spec.rows}x{spec.cols}x{spec.inner}"
        entry = shapes.setdefault(key, [0.0, 0, spec.flops()])
        entry[0] += mean_ms[i]
        entry[1] += 1
    per_shape = {k: round(v[2] / (v[0] / v[1] * 1e-3) / 1e12, 2) for k, v in shapes.items()}

    nn = layouts["NN"]
    nn_flops_per_launch = nn["flops"] / nn["launches"]
    nn_ms_per_launch = nn["ms"] / nn["launches"]
    achieved = nn_flops_per_launch / (nn_ms_per_launch * 1e-3) / 1e12
    roofline = {"kernel": "gemm_f32_kernel<Tile<128,128,16,2,2>, A k-contiguous, B n-contiguous> (all forward NN)",
                "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_FP32_TFLOPS, 4), "traffic": None,
                "launch_ms_mean": round(nn_ms_per_launch, 4), "flops_per_launch": nn_flops_per_launch}

    value = set_flops / (ms_per_step * 1e-3) / 1e12
    result = {
        "metric": "GEMM TFLOP/s and % fp32 MFMA peak (111.5M train set); decode GEMV GB/s, 1 GPU",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: seeded N(0,1) activations/gradients, N(0,0.02) weights, resident in HBM",
        "config": {"workload": "111.5M training GEMM set (config 2): 12 blocks x {qkv, out, up, down} x {NN, NT, TN}"
                               " + 16x1024 codebook head x {NN, NT, TN}, M=32768",
                   "gemms_per_step": len(calls), "tflop_per_step": round(set_flops / 1e12, 4)},
        "frac_fp32_peak": round(value / PEAK_FP32_TFLOPS, 4),
        "roofline": roofline,
        "per_layout": {k: {kk: round(vv, 4) for kk, vv in v.items()} for k, v in per_layout.items()},
        "per_shape_tflops": per_shape,
    }

    if not args.no_cpu:
        projected_s, sampled_flops, sampled_s, samples = cpu_baseline(gpu, calls, args.cpu_budget)
        result["cpu_baseline"] = {
            "value": round(set_flops / projected_s / 1e12, 8), "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"reference::matmul restated in C (oracle/), single thread, same input bytes; "
                      f"{sampled_flops / 1e9:.1f} GFLOP over row samples of the {len(samples)} distinct GEMMs "
                      f"({sampled_s:.1f} s), scaled linearly in rows to the full set: "
                      f"{projected_s:.0f} s per step",
            "host_cpu": _cpu_model(), "host_threads": os.cpu_count()}
    print(json.dumps(result))
    gpu.close()
    return 0


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


if __name__ == "__main__":
    sys.exit(main())
