"""Benchmark of the GEMM hot path on one MI355X.

Headline workload (the driver's metric, config 2): the 111.5M model's
training GEMM set, exactly as the reference's model issues it through
``Gpu::matmul``:
- 12 blocks x {QKV 768->2304, out-proj 768->768, FFN up 768->3072, FFN down 3072->768};
- plus the 16-codebook head 768->16384 (gpt.rs:72);
- each as forward NN (``Linear::forward``, linear.rs:43-48), input-gradient NT and
  weight-gradient TN with accumulate (``Linear::backward``, linear.rs:51-63);
- M = 16 x 2048 = 32768 tokens: 147 products, 19.173 TFLOP of algorithmic work per step.

Inputs are seeded synthetic data resident in HBM before timing (activations and
gradients ~N(0,1), weights ~N(0,0.02)). A "step" is one pass over that set, timed
with HIP events on the library's stream.

The printed JSON line is the driver's contract plus:
- ``roofline``: the forward-NN kernel, timed per launch with HIP events;
- ``cpu_baseline``: the reference's CPU matmul restated bit-for-bit in oracle/, on one
  host core, over a bounded row sample of every GEMM of the set, scaled to the full set
  (``cpu_baseline_all_cores``: the same with each sample's rows split over the host's cores);
- ``bf16``: the same set with bf16-rounded inputs and fp32 accumulation;
- ``attention``: config 3's six causal attention products, 192 heads x T = 2048 x h = 64;
- ``decode``: config 4's M in {1, 4, 16} products against the 111.5M weights, replayed
  from a HIP graph over a weight pool larger than the 256 MB Infinity Cache, and one
  decode token's 49 products in sequence;
- ``linear_bias``: config 2's Linear forward as the reference calls it (matmul, then
  add_row_bias) against the fused sn_matmul_bias, the bias-gradient column sums, and the weight
  and bias gradients as two calls (matmul, then accumulate_column_sums) against the one
  sn_matmul_column_sums call;
- ``head_cross_entropy``: the head's 16 per-codebook cross-entropy calls at config 2;
- ``published``: the reference's own published products (the only GEMM numbers it publishes, on
  Jetsons) with its timing method, fp32 and bf16; configs 0 and 1 as whole training sets; config 2's
  two weakest products;
- ``shard_of_8``: config 2's set at one GPU's share when its tokens are split over 8 GPUs (M = 4096).

``--vendor`` prints, instead, the same set through torch.mm (hipBLASLt / rocBLAS) beside this build's,
one decode token through torch.mm, and the shader clock under each set's load.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from staleynet_amd.gemm import BatchStrides, Gpu, MatmulSpec, Precision, Shape  # noqa: E402

# MI355X published peaks (dense): fp32 matrix 157.3 TFLOP/s, bf16 2.5 PFLOP/s, HBM 8 TB/s.
PEAK_FP32_TFLOPS = 157.3
PEAK_BF16_TFLOPS = 2500.0
PEAK_HBM_GBS = 8000.0
SEED = 1234
METRIC = "GEMM TFLOP/s and % fp32 MFMA peak (111.5M train set); decode GEMV GB/s, 1 GPU"


_HIP = None


def hip_runtime() -> ctypes.CDLL:
    """libamdhip64 with the signature of every entry point this file calls declared, so
    handles and sizes cross the ctypes boundary at their C widths (hipError_t results are
    C ints)."""
    global _HIP
    if _HIP is None:
        hip = ctypes.CDLL("libamdhip64.so")
        handle, handle_p = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
        signatures = {
            "hipEventCreate": [handle_p],
            "hipEventRecord": [handle, handle],
            "hipEventSynchronize": [handle],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), handle, handle],
            "hipEventDestroy": [handle],
            "hipDeviceSynchronize": [],
            "hipStreamBeginCapture": [handle, ctypes.c_int],
            "hipStreamEndCapture": [handle, handle_p],
            "hipGraphInstantiate": [handle_p, handle, handle_p, ctypes.c_char_p, ctypes.c_size_t],
            "hipGraphLaunch": [handle, handle],
            "hipGraphExecDestroy": [handle],
            "hipGraphDestroy": [handle],
        }
        for name, argtypes in signatures.items():
            function = getattr(hip, name)
            function.argtypes = argtypes
            function.restype = ctypes.c_int
        _HIP = hip
    return _HIP


class HipEvents:
    """hipEvent timing on an explicit stream (the library's own)."""

    def __init__(self):
        self.hip = hip_runtime()

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


class HipGraph:
    """Stream capture of a sequence of library calls into a HIP graph, so a
    launch-bound sequence (decode GEMVs) replays without per-call host cost.
    The library issues no memset or allocation inside sn_matmul, so every
    captured node is a kernel."""

    CAPTURE_RELAXED = 2

    def __init__(self, stream: int, record):
        hip = hip_runtime()
        self.hip, self.stream = hip, ctypes.c_void_p(stream)
        graph = ctypes.c_void_p()
        assert hip.hipStreamBeginCapture(self.stream, self.CAPTURE_RELAXED) == 0
        try:
            record()
        finally:
            assert hip.hipStreamEndCapture(self.stream, ctypes.byref(graph)) == 0
        self.graph = graph
        self.exec = ctypes.c_void_p()
        assert hip.hipGraphInstantiate(ctypes.byref(self.exec), graph, None, None, ctypes.c_size_t(0)) == 0

    def launch(self) -> None:
        assert self.hip.hipGraphLaunch(self.exec, self.stream) == 0

    def close(self) -> None:
        self.hip.hipGraphExecDestroy(self.exec)
        self.hip.hipGraphDestroy(self.graph)


class PlainReplay:
    """HipGraph's interface without a graph: `launch` issues the recorded calls directly. Used by
    --plain-launches, so that a profiled run captures no HIP graph."""

    def __init__(self, stream: int, record):
        self.record = record

    def launch(self) -> None:
        self.record()

    def close(self) -> None:
        pass


REPLAY = HipGraph


def timed(events: HipEvents, stream: int, body, repeats: int) -> float:
    """Milliseconds per repeat of `body`, events on `stream` around all repeats, after one
    untimed call (first launches of a kernel pay one-time loading costs)."""
    start, end = events.create(), events.create()
    body()
    events.device_synchronize()
    events.record(start, stream)
    for _ in range(repeats):
        body()
    events.record(end, stream)
    ms = events.elapsed_ms(start, end) / repeats
    events.destroy(start)
    events.destroy(end)
    return ms


# ---- the training GEMM set ------------------------------------------------------------

MODEL_111M = dict(name="111.5M", blocks=12, width=768, ffn=3072, heads_width=16 * 1024, tokens=16 * 2048)


def linear_products(tokens: int, inputs: int, outputs: int):
    """The three products of one Linear (linear.rs:43-63): forward NN, dW TN (accumulate), dX NT."""
    return [
        ("NN", MatmulSpec.new(tokens, outputs, inputs)),
        ("TN", MatmulSpec.new(inputs, outputs, tokens).left_transposed().accumulate()),
        ("NT", MatmulSpec.new(tokens, inputs, outputs).right_transposed()),
    ]


def training_set(model=MODEL_111M):
    """(label, inputs, outputs) for every Linear of one training step."""
    d, f = model["width"], model["ffn"]
    layers = [("qkv", d, 3 * d), ("out", d, d), ("up", d, f), ("down", f, d)]
    items = [(f"b{block}.{name}", i, o) for block in range(model["blocks"]) for name, i, o in layers]
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
    calls, buffers = [], []
    for index, (label, inputs, outputs) in enumerate(training_set(model)):
        buf = LinearBuffers(gpu, model["tokens"], inputs, outputs, 16 * index)
        buffers.append(buf)
        for layout, spec in linear_products(model["tokens"], inputs, outputs):
            calls.append((label, layout, spec, buf.operands(layout)))
    gpu.synchronize()
    return calls, buffers


def run_step(gpu: Gpu, calls, precision=Precision.Default, events=None, marks=None, stream=0):
    for i, (_, _, spec, (left, right, out)) in enumerate(calls):
        if marks is not None:
            events.record(marks[i], stream)
        gpu.matmul(spec.with_precision(precision) if precision else spec, left, right, out)
    if marks is not None:
        events.record(marks[len(calls)], stream)


def measure_set(gpu: Gpu, events: HipEvents, calls, steps: int, warmup: int, precision=Precision.Default):
    """Step time over `steps` steps and per-launch times from events between launches."""
    stream = gpu.stream
    for _ in range(warmup):
        run_step(gpu, calls, precision)
    events.device_synchronize()
    marks = [[events.create() for _ in range(len(calls) + 1)] for _ in range(steps)]
    start, end = events.create(), events.create()
    events.record(start, stream)
    for step in range(steps):
        run_step(gpu, calls, precision, events, marks[step], stream)
    events.record(end, stream)
    events.device_synchronize()
    ms_per_step = events.elapsed_ms(start, end) / steps
    per_call = np.array([[events.elapsed_ms(marks[s][i], marks[s][i + 1]) for i in range(len(calls))]
                         for s in range(steps)]).mean(axis=0)
    for row in marks:
        for e in row:
            events.destroy(e)
    return ms_per_step, per_call


def replayed_step_ms(gpu: Gpu, events: HipEvents, calls, steps: int, precision=Precision.Default) -> float:
    """Milliseconds per step with the step's calls captured once into a HIP graph and replayed:
    the kernels back to back without the host's per-call cost (ctypes, and the events that
    measure_set records between launches), which sets the rate of sets of short products."""
    graph = REPLAY(gpu.stream, lambda: run_step(gpu, calls, precision))
    try:
        return timed(events, gpu.stream, graph.launch, steps)
    finally:
        graph.close()


def summarize_set(calls, per_call_ms, peak):
    layouts, shapes = {}, {}
    for i, (_, layout, spec, _) in enumerate(calls):
        entry = layouts.setdefault(layout, {"flops": 0, "ms": 0.0, "launches": 0})
        entry["flops"] += spec.flops()
        entry["ms"] += per_call_ms[i]
        entry["launches"] += 1
        key = f"{layout} {spec.rows}x{spec.cols}x{spec.inner}"
        s = shapes.setdefault(key, [0.0, 0, spec.flops()])
        s[0] += per_call_ms[i]
        s[1] += 1
    per_layout = {k: {"tflops": round(v["flops"] / (v["ms"] * 1e-3) / 1e12, 2), "ms_per_step": round(v["ms"], 3),
                      "frac_peak": round(v["flops"] / (v["ms"] * 1e-3) / 1e12 / peak, 4)}
                  for k, v in layouts.items()}
    per_shape = {k: round(v[2] / (v[0] / v[1] * 1e-3) / 1e12, 1) for k, v in shapes.items()}
    return layouts, per_layout, per_shape


def bf16_roofline_tflops(spec: MatmulSpec) -> float:
    """min(bf16 dense peak, algorithmic intensity x HBM bandwidth) with fp32 operands in HBM."""
    m, n, k = spec.rows, spec.cols, spec.inner
    bytes_moved = 4 * (m * k + k * n + m * n * (2 if spec.write else 1))
    return min(PEAK_BF16_TFLOPS, spec.flops() / bytes_moved * PEAK_HBM_GBS / 1e3)


# ---- config 3: causal attention ---------------------------------------------------------

def backward_products(heads: int, t: int, h: int, workspace: int = 1536 << 20) -> int:
    """Products' MFMAs per visible pair that sn_causal_attention_backward executes on a causal
    [heads, t, t] problem with the default workspace: 5 when dQ's partial sums (h floats per query
    and 128-key block that reaches it) fit after the 12-byte row records (head dims 32 and 64),
    else 7 (the query kernel recomputes S and dP)."""
    records = (heads * 3 * ((t + 3) // 4 * 4) * 4 + 255) // 256 * 256
    rows = sum(t - b * 128 // 64 * 64 for b in range((t + 127) // 128))
    return 5 if h <= 64 and records + heads * rows * h * 4 <= workspace else 7


def measure_attention(gpu: Gpu, events: HipEvents, repeats: int = 3):
    """The six attention products of attention.rs:206-260 for 16 x 12 heads, T = 2048, h = 64,
    dense (the reference's calls) and with the causal-mask extension."""
    heads, t, h = 16 * 12, 2048, 64
    head_block, score_block = t * h, t * t
    per_head = lambda l, r, o: BatchStrides(heads, l, r, o)  # noqa: E731
    q, k, v, do = (gpu.zeros(Shape(heads * t, h)) for _ in range(4))
    p, ds = gpu.zeros(Shape(heads * t, t)), gpu.zeros(Shape(heads * t, t))
    for i, tensor in enumerate((q, k, v, do, p, ds)):
        gpu.fill_normal(tensor, SEED, 900 + i)
    s_out, dp_out = gpu.zeros(Shape(heads * t, t)), gpu.zeros(Shape(heads * t, t))
    o, dv, dq, dk = (gpu.zeros(Shape(heads * t, h)) for _ in range(4))
    scores = MatmulSpec.new(t, t, h).right_transposed().batched(per_head(head_block, head_block, score_block))
    mix = MatmulSpec.new(t, h, t).batched(per_head(score_block, head_block, head_block))
    transposed_mix = MatmulSpec.new(t, h, t).left_transposed().batched(per_head(score_block, head_block, head_block))
    products = [
        ("scores Q.K^T", scores, q, k, s_out, "out"),
        ("mix P.V", mix, p, v, o, "left"),
        ("dP = dO.V^T", scores, do, v, dp_out, "out"),
        ("dV = P^T.dO", transposed_mix, p, do, dv, "left"),
        ("dQ = s.dS.K", mix.scaled(0.125), ds, k, dq, "left"),
        ("dK = s.dS^T.Q", transposed_mix.scaled(0.125), ds, q, dk, "left"),
    ]
    causal_flops = 2 * h * t * (t + 1) // 2 * heads  # visible (q, k) pairs only
    dense_flops = 2 * h * t * t * heads
    result = {"shape": "16x12 heads, T=2048, h=64, fp32", "causal_gflop_per_product": round(causal_flops / 1e9, 2),
              "products": {}}
    total = {"dense": 0.0, "causal": 0.0}
    for name, spec, left, right, out, kind in products:
        masked = spec.causal_output() if kind == "out" else spec.causal_left()
        dense_ms = timed(events, gpu.stream, lambda: gpu.matmul(spec, left, right, out), repeats)
        causal_ms = timed(events, gpu.stream, lambda: gpu.matmul(masked, left, right, out), repeats)
        total["dense"] += dense_ms
        total["causal"] += causal_ms
        result["products"][name] = {
            "dense_ms": round(dense_ms, 3), "dense_tflops": round(dense_flops / (dense_ms * 1e-3) / 1e12, 1),
            "causal_ms": round(causal_ms, 3),
            "causal_tflops_on_visible_work": round(causal_flops / (causal_ms * 1e-3) / 1e12, 1)}
    result["all_six"] = {"dense_ms": round(total["dense"], 3), "causal_ms": round(total["causal"], 3),
                         "causal_tflops_on_visible_work": round(6 * causal_flops / (total["causal"] * 1e-3) / 1e12, 1),
                         "dense_tflops": round(6 * dense_flops / (total["dense"] * 1e-3) / 1e12, 1)}
    # The row-wise kernels between the products (attention.rs:210, :249), on the same 192 x 2048 x
    # 2048 matrices: causal_softmax reads each visible score and writes every element (4 bytes
    # each); softmax_backward reads P and dP and writes dS (12 bytes per element).
    visible = heads * t * (t + 1) // 2
    gpu.copy_device(p, s_out)
    softmax_ms = timed(events, gpu.stream, lambda: gpu.causal_softmax(s_out, t, 0.125, 0), repeats)
    gpu.causal_softmax(p, t, 0.125, 0)
    backward_ms = timed(events, gpu.stream, lambda: gpu.softmax_backward(p, dp_out), repeats)
    result["row_kernels"] = {
        "causal_softmax_ms": round(softmax_ms, 3),
        "causal_softmax_gbs": round(4 * (visible + heads * t * t) / (softmax_ms * 1e-3) / 1e9, 1),
        "softmax_backward_ms": round(backward_ms, 3),
        "softmax_backward_gbs": round(12 * heads * t * t / (backward_ms * 1e-3) / 1e9, 1)}
    # The head permutes around them (layers/attention.rs:202-214): Q, K and V split out of the packed
    # [16 x 2048, 3 x 768] QKV projection into head-major [192 x 2048, 64], and the context merged
    # back into [16 x 2048, 768]; 8 bytes per moved element.
    from staleynet_amd.gemm import HeadLayout
    packed = gpu.zeros(Shape(16 * t, 3 * 12 * h))
    gpu.fill_normal(packed, SEED, 950)
    layouts = [HeadLayout.dense(16, t, 12, h, 3 * 12 * h, part * 12 * h) for part in range(3)]
    split_ms = timed(events, gpu.stream, lambda: [gpu.split_heads(packed, dst, lay)
                                                  for dst, lay in zip((q, k, v), layouts)], repeats)
    merge_ms = timed(events, gpu.stream, lambda: gpu.merge_heads(o, packed, layouts[0]), repeats)
    moved = heads * t * h
    result["row_kernels"].update({
        "split_qkv_ms": round(split_ms, 3), "split_qkv_gbs": round(3 * 8 * moved / (split_ms * 1e-3) / 1e9, 1),
        "merge_ms": round(merge_ms, 3), "merge_gbs": round(8 * moved / (merge_ms * 1e-3) / 1e9, 1)})
    packed.free()
    result["step_ms"] = {"products_causal": round(total["causal"], 3),
                         "with_row_kernels": round(total["causal"] + softmax_ms + backward_ms + split_ms + merge_ms, 3)}
    # The fused forward (sn_causal_attention) against the three calls it replaces (scores
    # product, causal_softmax, mix product): O only, and O with the probabilities the backward
    # reads. FLOPs on the visible (query, key) pairs: two products of 2 h per pair.
    unfused_ms = (result["products"]["scores Q.K^T"]["causal_ms"] + softmax_ms
                  + result["products"]["mix P.V"]["causal_ms"])
    fused_ms = timed(events, gpu.stream, lambda: gpu.causal_attention(q, k, v, o, heads, t, t, h, 0.125), repeats)
    fused_p_ms = timed(events, gpu.stream, lambda: gpu.causal_attention(q, k, v, o, heads, t, t, h, 0.125,
                                                                        probabilities=p), repeats)
    # The fused probability gradient against the dP product (causal mask) and softmax_backward.
    unfused_grad_ms = result["products"]["dP = dO.V^T"]["causal_ms"] + backward_ms
    gpu.causal_attention(q, k, v, o, heads, t, t, h, 0.125, probabilities=p)
    fused_grad_ms = timed(events, gpu.stream, lambda: gpu.causal_attention_score_grad(do, v, o, p, ds, heads, t, t, h),
                          repeats)
    # ... and with the query gradient (dQ = scale dS K) accumulated in the same launch.
    unfused_grad_q_ms = unfused_grad_ms + result["products"]["dQ = s.dS.K"]["causal_ms"]
    fused_grad_q_ms = timed(events, gpu.stream, lambda: gpu.causal_attention_score_grad(
        do, v, o, p, ds, heads, t, t, h, k=k, q_grad=dq, scale=0.125), repeats)
    result["fused_score_grad"] = {"dp_and_softmax_backward_ms": round(unfused_grad_ms, 3),
                                  "fused_ms": round(fused_grad_ms, 3),
                                  "dp_softmax_backward_and_dq_ms": round(unfused_grad_q_ms, 3),
                                  "fused_with_dq_ms": round(fused_grad_q_ms, 3)}
    result["fused_forward"] = {
        "three_calls_ms": round(unfused_ms, 3), "fused_ms": round(fused_ms, 3),
        "fused_with_probabilities_ms": round(fused_p_ms, 3),
        "fused_tflops_on_visible_work": round(2 * causal_flops / (fused_ms * 1e-3) / 1e12, 1)}
    # One layer's attention training kernels, two ways. Keeping P: the fused forward with the
    # probabilities, the fused score gradient with dQ, and the causal dV and dK products. Without
    # P (sn_causal_attention_with_stats + sn_causal_attention_backward): the forward keeps 8
    # bytes per query, the backward recomputes S and dP once (5 products' MFMAs over the visible
    # pairs against the reference's 4) with dQ's partial sums per key block in the context's
    # workspace (855 MB here, of 1.5 GiB), or twice (7) where they do not fit.
    keeping_p_ms = (fused_p_ms + fused_grad_q_ms + result["products"]["dV = P^T.dO"]["causal_ms"]
                    + result["products"]["dK = s.dS^T.Q"]["causal_ms"])
    stats = gpu.zeros(Shape.vector(2 * heads * t))
    stats_ms = timed(events, gpu.stream, lambda: gpu.causal_attention_with_stats(q, k, v, o, stats, heads, t, t, h,
                                                                                 0.125), repeats)
    backward_p_free_ms = timed(events, gpu.stream, lambda: gpu.causal_attention_backward(
        q, k, v, o, do, stats, dq, dk, dv, heads, t, t, h, 0.125), repeats)
    stats.free()
    result["training_kernels"] = {
        "keeping_probabilities_ms": round(keeping_p_ms, 3),
        "probability_free_ms": round(stats_ms + backward_p_free_ms, 3),
        "forward_with_stats_ms": round(stats_ms, 3), "backward_ms": round(backward_p_free_ms, 3),
        "backward_tflops_on_reference_work": round(4 * causal_flops / (backward_p_free_ms * 1e-3) / 1e12, 1),
        "backward_tflops_executed": round(backward_products(heads, t, h) * causal_flops / (backward_p_free_ms * 1e-3)
                                          / 1e12, 1),
        "probability_bytes_not_kept": 4 * heads * t * t}
    return result


def run_one_attention(gpu: Gpu, events: HipEvents, kind: str) -> dict:
    """Config 3's fused attention kernel alone (192 heads, T = 2048, h = 64), one warm-up and five
    timed calls: `forward` (O only), `forward_p` (O and the probabilities), `score_grad` (dS from
    dO, V, O, P), `score_grad_dq` (with dQ), `forward_stats` (O and the row statistics) or
    `backward` (dQ, dK, dV from the statistics, no P): the workload of the attention counter
    profiles."""
    heads, t, h = 16 * 12, 2048, 64
    q, k, v, o, do, dq = (gpu.zeros(Shape(heads * t, h)) for _ in range(6))
    p, ds = gpu.zeros(Shape(heads * t, t)), gpu.zeros(Shape(heads * t, t))
    for i, tensor in enumerate((q, k, v, do)):
        gpu.fill_normal(tensor, SEED, 900 + i)
    dk, dv = gpu.zeros(Shape(heads * t, h)), gpu.zeros(Shape(heads * t, h))
    stats = gpu.zeros(Shape.vector(2 * heads * t))
    if kind.startswith("score_grad"):  # the gradient reads the forward's O and P
        gpu.causal_attention(q, k, v, o, heads, t, t, h, 0.125, probabilities=p)
    if kind == "backward":  # ... this one O and the statistics
        gpu.causal_attention_with_stats(q, k, v, o, stats, heads, t, t, h, 0.125)
    calls = {
        "forward": lambda: gpu.causal_attention(q, k, v, o, heads, t, t, h, 0.125),
        "forward_p": lambda: gpu.causal_attention(q, k, v, o, heads, t, t, h, 0.125, probabilities=p),
        "score_grad": lambda: gpu.causal_attention_score_grad(do, v, o, p, ds, heads, t, t, h),
        "score_grad_dq": lambda: gpu.causal_attention_score_grad(do, v, o, p, ds, heads, t, t, h, k=k, q_grad=dq,
                                                                 scale=0.125),
        "forward_stats": lambda: gpu.causal_attention_with_stats(q, k, v, o, stats, heads, t, t, h, 0.125),
        "backward": lambda: gpu.causal_attention_backward(q, k, v, o, do, stats, dq, dk, dv, heads, t, t, h, 0.125),
    }
    ms = timed(events, gpu.stream, calls[kind], 5)
    visible = heads * t * (t + 1) // 2
    # The reference's products the call stands for (the backward executes 7 products' MFMAs for its 4).
    products = {"forward": 2, "forward_p": 2, "score_grad": 1, "score_grad_dq": 2, "forward_stats": 2,
                "backward": 4}[kind]
    return {"attention": kind, "ms": round(ms, 4),
            "tflops_on_visible_work": round(products * 2 * h * visible / (ms * 1e-3) / 1e12, 1)}


# ---- config 4: decode ------------------------------------------------------------------

DECODE_SHAPES = [("qkv", 768, 2304), ("out", 768, 768), ("up", 768, 3072), ("down", 3072, 768),
                 ("head", 768, 16 * 1024)]


def decode_bytes(m: int, k: int, n: int) -> int:
    """Algorithmic bytes of one decode product: read W and x, write y (fp32)."""
    return 4 * (k * n + m * k + m * n)


def measure_decode(gpu: Gpu, events: HipEvents, pool_bytes: int = 640 << 20, repeats: int = 3):
    """GB/s of y[M,N] = x[M,K] W[K,N] per shape, W drawn from a pool larger than the
    256 MB Infinity Cache so reads come from HBM; launches replayed from a HIP graph.
    Then one token's sequence (12 blocks x 4 products + head, distinct weights, M = 1)."""
    result = {"per_shape_gbs": {}, "method": "HIP-graph replay, fp32 weights rotated through a "
              f"{pool_bytes >> 20} MB pool (> 256 MB MALL); bytes = 4(KN + MK + MN)"}
    # Practical read roofline: a plain streaming read (sn_read_sum) of 2 GiB.
    src, sums = gpu.zeros(Shape(1 << 29, 1)), gpu.zeros(Shape(8192, 1))
    gpu.read_sum(src, sums)
    ms = timed(events, gpu.stream, lambda: gpu.read_sum(src, sums), 5)
    result["stream_read_gbs"] = round((1 << 31) / (ms * 1e-3) / 1e9, 1)
    src.free()
    # The same streaming read, one launch per head-sized (50.3 MB) buffer rotated through the
    # pool and replayed from a HIP graph: the practical ceiling of a single launch that reads
    # the head's weight once (launch, ramp-up and drain included). Best of 3 grid sizes.
    head_k, head_n = DECODE_SHAPES[4][1], DECODE_SHAPES[4][2]
    copies = max(2, -(-pool_bytes // (4 * head_k * head_n)))
    pool = [gpu.zeros(Shape(head_k, head_n)) for _ in range(copies)]
    best = 0.0
    for blocks in (1024, 2048, 4096):
        part = gpu.zeros(Shape(blocks, 1))
        graph = REPLAY(gpu.stream, lambda: [gpu.read_sum(w, part) for w in pool])
        graph.launch()
        ms = timed(events, gpu.stream, graph.launch, repeats) / copies
        graph.close()
        part.free()
        best = max(best, 4 * head_k * head_n / (ms * 1e-3) / 1e9)
    for w in pool:
        w.free()
    sums.free()
    result["stream_read_head_size_gbs"] = round(best, 1)
    # A plain streaming read of each weight, one launch per weight of the same kind of pool: the
    # ceiling a single launch reading that many bytes reaches here (best of three grid sizes).
    result["read_same_weight_us"] = {}
    for name, k, n in DECODE_SHAPES:
        copies = max(2, -(-pool_bytes // (4 * k * n)))
        pool = [gpu.zeros(Shape(k, n)) for _ in range(copies)]
        best_ms = None
        for blocks in (256, 512, 1024):
            part = gpu.zeros(Shape(blocks, 1))
            graph = REPLAY(gpu.stream, lambda: [gpu.read_sum(w, part) for w in pool])
            graph.launch()
            ms = timed(events, gpu.stream, graph.launch, repeats) / copies
            graph.close()
            part.free()
            best_ms = ms if best_ms is None else min(best_ms, ms)
        for w in pool:
            w.free()
        result["read_same_weight_us"][f"{name} {k}x{n}"] = round(best_ms * 1e3, 2)
    result["per_shape_us"] = {}
    for m in (1, 4, 16):
        for name, k, n in DECODE_SHAPES:
            copies = max(2, -(-pool_bytes // (4 * k * n)))
            pool = [gpu.zeros(Shape(k, n)) for _ in range(copies)]
            for i, w in enumerate(pool):
                gpu.fill_normal(w, SEED, 1000 + i, 0.0, 0.02)
            x, y = gpu.zeros(Shape(m, k)), gpu.zeros(Shape(m, n))
            gpu.fill_normal(x, SEED, 999)
            spec = MatmulSpec.new(m, n, k)
            graph = REPLAY(gpu.stream, lambda: [gpu.matmul(spec, x, w, y) for w in pool])
            graph.launch()
            ms = timed(events, gpu.stream, graph.launch, repeats) / copies
            graph.close()
            result["per_shape_gbs"][f"M={m} {name} {k}x{n}"] = round(decode_bytes(m, k, n) / (ms * 1e-3) / 1e9, 1)
            result["per_shape_us"][f"M={m} {name} {k}x{n}"] = round(ms * 1e3, 2)
            for w in pool:
                w.free()
    # One decode token: every product of the 12 blocks and the head, each weight distinct.
    layers = [(k, n) for _ in range(12) for _, k, n in DECODE_SHAPES[:4]] + [DECODE_SHAPES[4][1:]]
    weights = []
    for i, (k, n) in enumerate(layers):
        w = gpu.zeros(Shape(k, n))
        gpu.fill_normal(w, SEED, 2000 + i, 0.0, 0.02)
        weights.append((w, gpu.zeros(Shape(1, k)), gpu.zeros(Shape(1, n)), MatmulSpec.new(1, n, k)))
    token_bytes = sum(decode_bytes(1, k, n) for k, n in layers)
    graph = REPLAY(gpu.stream, lambda: [gpu.matmul(spec, x, w, y) for w, x, y, spec in weights])
    graph.launch()
    ms = timed(events, gpu.stream, graph.launch, 5)
    graph.close()
    # What bounds the layer products: the per-launch floor (the smallest product, replayed 96 times)
    # and the same products with their weight resident in the Infinity Cache (96 launches over two
    # weights) against the HBM-resident rates above.
    x, w, y = gpu.zeros(Shape(1, 4)), gpu.zeros(Shape(4, 64)), gpu.zeros(Shape(1, 64))
    tiny = MatmulSpec.new(1, 64, 4)
    graph = REPLAY(gpu.stream, lambda: [gpu.matmul(tiny, x, w, y) for _ in range(96)])
    graph.launch()
    result["launch_floor_us"] = round(timed(events, gpu.stream, graph.launch, repeats) / 96 * 1e3, 2)
    graph.close()
    for t in (x, w, y):
        t.free()
    result["cache_resident_us"] = {}
    for name, k, n in DECODE_SHAPES:
        pair = [gpu.zeros(Shape(k, n)) for _ in range(2)]
        x, y = gpu.zeros(Shape(1, k)), gpu.zeros(Shape(1, n))
        spec = MatmulSpec.new(1, n, k)
        graph = REPLAY(gpu.stream, lambda: [gpu.matmul(spec, x, pair[i % 2], y) for i in range(96)])
        graph.launch()
        result["cache_resident_us"][f"M=1 {name} {k}x{n}"] = round(timed(events, gpu.stream, graph.launch, repeats)
                                                                   / 96 * 1e3, 2)
        graph.close()
        for t in pair + [x, y]:
            t.free()
    result["attention"] = measure_decode_attention(gpu, events, repeats)
    head = result["per_shape_gbs"][f"M=1 head {DECODE_SHAPES[4][1]}x{DECODE_SHAPES[4][2]}"]
    result["head_m1_frac_hbm_peak"] = round(head / PEAK_HBM_GBS, 4)
    result["head_m1_frac_stream_read"] = round(head / result["stream_read_gbs"], 4)
    result["head_m1_frac_stream_read_head_size"] = round(head / result["stream_read_head_size_gbs"], 4)
    result["m1_over_read_same_weight"] = {
        f"{name} {k}x{n}": round(result["per_shape_us"][f"M=1 {name} {k}x{n}"]
                                 / result["read_same_weight_us"][f"{name} {k}x{n}"], 2)
        for name, k, n in DECODE_SHAPES}
    result["token_sequence"] = {"products": len(layers), "mb_per_token": round(token_bytes / 1e6, 1),
                                "us_per_token": round(ms * 1e3, 1),
                                "gbs": round(token_bytes / (ms * 1e-3) / 1e9, 1)}
    return result


def measure_decode_attention(gpu: Gpu, events: HipEvents, repeats: int = 3):
    """One decode step's attention per layer of the 111.5M model (attention.rs:274-320): 12 heads,
    one new position against a 1408-position KV cache holding `cached` positions. The reference's
    three calls (scores product against the cache, causal_softmax, mix product; causal masks from the
    query offset) against the fused sn_causal_attention, whose few-query form splits the cached keys
    over workgroups; each replayed 12 times from a HIP graph, microseconds per layer."""
    heads, capacity, h = 12, 1408, 64
    q, o = gpu.zeros(Shape(heads, h)), gpu.zeros(Shape(heads, h))
    k, v = gpu.zeros(Shape(heads * capacity, h)), gpu.zeros(Shape(heads * capacity, h))
    scores = gpu.zeros(Shape(heads, capacity))
    for i, t in enumerate((q, k, v)):
        gpu.fill_normal(t, SEED, 960 + i)
    out = {"shape": f"{heads} heads, 1 query, cache {capacity} x {h}, fp32", "method": "HIP-graph replay x12"}
    for cached in (701, capacity):
        offset = cached - 1
        fused = lambda: gpu.causal_attention(q, k, v, o, heads, 1, capacity, h, 0.125,  # noqa: E731
                                             query_offset=offset, q_stride=h, kv_stride=capacity * h)
        per_head = BatchStrides(heads, h, capacity * h, capacity)
        score_spec = MatmulSpec.new(1, capacity, h).right_transposed().batched(per_head).causal_output(offset)
        mix_spec = MatmulSpec.new(1, h, capacity).batched(BatchStrides(heads, capacity, capacity * h, h)) \
            .causal_left(offset)

        def three_calls():
            gpu.matmul(score_spec, q, k, scores)
            gpu.causal_softmax(scores, 1, 0.125, offset)
            gpu.matmul(mix_spec, scores, v, o)

        for name, body in (("fused_us", fused), ("three_calls_us", three_calls)):
            graph = REPLAY(gpu.stream, lambda: [body() for _ in range(12)])
            graph.launch()
            ms = timed(events, gpu.stream, graph.launch, repeats) / 12
            graph.close()
            out.setdefault(f"cached={cached}", {})[name] = round(ms * 1e3, 2)
    for t in (q, o, k, v, scores):
        t.free()
    return out


DECODE_PMC_POOL_BYTES = 640 << 20
DECODE_PMC_MEASURED = 8


def _decode_pmc_launches(pool_bytes: int = DECODE_PMC_POOL_BYTES, measured: int = DECODE_PMC_MEASURED):
    """(m, name, k, n, weight index, measured) of every decode product the counter workload
    launches, in launch order, without a GPU: per shape one pass over a weight pool larger than
    the 256 MB Infinity Cache, then `measured` more products on the pool's first weights, each
    last read about pool_bytes earlier, so their reads come from HBM."""
    for m in (1, 4, 16):
        for name, k, n in DECODE_SHAPES:
            copies = max(2, -(-pool_bytes // (4 * k * n)))
            for i in range(copies):
                yield m, name, k, n, i, False
            for i in range(measured):
                yield m, name, k, n, i % copies, True


def run_decode_pmc_workload(gpu: Gpu) -> int:
    """The decode products of _decode_pmc_launches, one plain launch each (no graph, so every
    dispatch is its own counter sample and trace record)."""
    launches = list(_decode_pmc_launches())
    current, pool, x, y = None, [], None, None
    for m, name, k, n, i, _ in launches:
        if current != (m, name):
            for t in pool + [x, y]:
                if t is not None:
                    t.free()
            copies = max(2, -(-DECODE_PMC_POOL_BYTES // (4 * k * n)))
            pool = [gpu.zeros(Shape(k, n)) for _ in range(copies)]
            for j, w in enumerate(pool):
                gpu.fill_normal(w, SEED, 1000 + j, 0.0, 0.02)
            x, y = gpu.zeros(Shape(m, k)), gpu.zeros(Shape(m, n))
            gpu.fill_normal(x, SEED, 999)
            spec = MatmulSpec.new(m, n, k)
            current = (m, name)
        gpu.matmul(spec, x, pool[i], y)
    gpu.synchronize()
    for t in pool + [x, y]:
        t.free()
    return len(launches)


DECODE_ATTENTION = dict(heads=12, capacity=1408, head_dim=64, cached=701)


def decode_attention_bytes(kind: str, heads: int, capacity: int, h: int, visible: int) -> int:
    """Algorithmic bytes of one decode-attention launch (one query per head, `visible` cached keys):
    the fused form reads q and the visible K and V rows and writes o; the reference's three calls
    are the scores product (q, visible K rows in; the whole [heads, capacity] score row out),
    causal_softmax (visible scores in, the whole row out) and the mix (visible P and V rows in, o out)."""
    return 4 * {"fused": 2 * heads * visible * h + 2 * heads * h,
                "scores": heads * visible * h + heads * h + heads * capacity,
                "softmax": heads * visible + heads * capacity,
                "mix": heads * visible + heads * visible * h + heads * h}[kind]


def run_decode_attention_pmc_workload(gpu: Gpu, pool_bytes: int = DECODE_PMC_POOL_BYTES) -> int:
    """One decode step's attention (12 heads, one query against a 1408-position cache holding 701)
    over a pool of distinct caches larger than the 256 MB Infinity Cache, one plain launch per call:
    the fused decode form over the whole pool, then the reference's three calls over it."""
    a = DECODE_ATTENTION
    heads, capacity, h, offset = a["heads"], a["capacity"], a["head_dim"], a["cached"] - 1
    copies = max(2, -(-pool_bytes // (8 * heads * capacity * h)))
    caches = []
    for i in range(copies):
        k, v = gpu.zeros(Shape(heads * capacity, h)), gpu.zeros(Shape(heads * capacity, h))
        gpu.fill_normal(k, SEED, 6000 + 2 * i)
        gpu.fill_normal(v, SEED, 6001 + 2 * i)
        caches.append((k, v))
    q, o = gpu.zeros(Shape(heads, h)), gpu.zeros(Shape(heads, h))
    scores = gpu.zeros(Shape(heads, capacity))
    gpu.fill_normal(q, SEED, 5999)
    score_spec = MatmulSpec.new(1, capacity, h).right_transposed().batched(
        BatchStrides(heads, h, capacity * h, capacity)).causal_output(offset)
    mix_spec = MatmulSpec.new(1, h, capacity).batched(BatchStrides(heads, capacity, capacity * h, h)).causal_left(offset)
    for k, v in caches:
        gpu.causal_attention(q, k, v, o, heads, 1, capacity, h, 0.125, query_offset=offset, q_stride=h,
                             kv_stride=capacity * h)
    for k, v in caches:
        gpu.matmul(score_spec, q, k, scores)
        gpu.causal_softmax(scores, 1, 0.125, offset)
        gpu.matmul(mix_spec, scores, v, o)
    gpu.synchronize()
    for t in [q, o, scores] + [t for pair in caches for t in pair]:
        t.free()
    return 4 * copies


def summarize_kernel_pmc(fetch_csv: str, write_csv: str, trace_csv: str, copy_mib: int, algorithmic: dict) -> str:
    """Per kernel (name holding a key of `algorithmic`, bytes per launch): mean HBM read and write
    bytes per dispatch (FETCH_SIZE, WRITE_SIZE, copy-calibrated as in summarize_pmc) and mean
    duration from a kernel-trace run of the same workload."""
    fetch, write = _per_dispatch(fetch_csv, "FETCH_SIZE"), _per_dispatch(write_csv, "WRITE_SIZE")
    copy_bytes = copy_mib << 20
    pick = lambda table, key: next(v for k, v in table.items() if key in k)  # noqa: E731
    f_factor = pick(fetch, COPY_KERNEL_KEY)[-1] * 1024 / copy_bytes
    w_factor = pick(write, COPY_KERNEL_KEY)[-1] * 1024 / copy_bytes
    lines = [f"copy kernel ({copy_mib} MiB read + {copy_mib} MiB written): factors {f_factor:.4f} (fetch), "
             f"{w_factor:.4f} (write)", "",
             f"{'kernel':>28} {'launches':>8} {'alg KB':>8} {'HBM rd KB':>10} {'HBM wr KB':>10} "
             f"{'traffic/alg':>11} {'kernel us':>10} {'alg GB/s':>9} {'HBM GB/s':>9}"]
    for key, alg in algorithmic.items():
        f = [v for name, values in fetch.items() if key in name for v in values]
        w = [v for name, values in write.items() if key in name for v in values]
        ns = _trace_durations(trace_csv, key)
        if not f or not w or not ns:
            continue
        rd = sum(f) / len(f) * 1024 / f_factor
        wr = sum(w) / len(w) * 1024 / w_factor
        t = sum(ns) / len(ns)
        lines.append(f"{key:>28} {len(ns):>8} {alg / 1e3:>8.1f} {rd / 1e3:>10.1f} {wr / 1e3:>10.1f} "
                     f"{(rd + wr) / alg:>11.3f} {t / 1e3:>10.2f} {alg / t:>9.0f} {(rd + wr) / t:>9.0f}")
    return "\n".join(lines)


def decode_attention_algorithmic() -> dict:
    a = DECODE_ATTENTION
    args = (a["heads"], a["capacity"], a["head_dim"], a["cached"])
    return {"decode_attention_kernel": decode_attention_bytes("fused", *args),
            "gemv_nt_kernel": decode_attention_bytes("scores", *args),
            "causal_softmax": decode_attention_bytes("softmax", *args),
            "gemv_kernel": decode_attention_bytes("mix", *args)}


# ---- the reference's published shapes, configs 0 and 1, the weakest config-2 products ------

# The only GEMM numbers the reference publishes (book/src/experiments.md:50-52, paper/appendix.tex:49-51,
# paper/body.tex:1261-1263): row-major NN forward products timed by `staleynet bench`
# (crates/staleynet-cli/src/commands/bench.rs:131-140), on NVIDIA Jetsons. (label, M, N, K,
# Orin NX register-blocked GFLOP/s, AGX Thor TF32 tensor-core GFLOP/s.)
PUBLISHED = [
    ("QKV projection", 2048, 768, 256, 579.0, 929.0),
    ("FFN expand", 2048, 1024, 256, 450.6, 730.0),
    ("output heads (4 codebooks)", 2048, 4096, 256, 458.5, 970.0),
]
MODEL_7M = dict(name="7.1M", blocks=6, width=256, ffn=1024, heads_width=16 * 1024, tokens=4 * 512)
MODEL_43M = dict(name="42.9M", blocks=8, width=512, ffn=2048, heads_width=16 * 1024, tokens=8 * 1024)


def reference_method_ms(events: HipEvents, stream: int, body) -> float:
    """The reference's bench timing (bench.rs:117-128; experiments.md:42-47): the mean of 5 runs
    after 1 warm-up, and the median of 3 such measurements."""
    return sorted(timed(events, stream, body, 5) for _ in range(3))[1]


def measure_published(gpu: Gpu, events: HipEvents, set_per_shape: dict):
    """The reference's published products on one MI355X, fp32 and bf16, beside the Jetson figures
    (context only: other hardware, and the reference benches zero-filled operands where these are
    seeded); configs 0 and 1 as whole training sets; config 2's two weakest products."""
    result = {"method": "mean of 5 launches after 1 warm-up, median of 3 (bench.rs:117-128); GFLOP/s = 2MNK/t",
              "products": {}}
    for label, m, n, k, orin, thor in PUBLISHED:
        x, w, y = gpu.zeros(Shape(m, k)), gpu.zeros(Shape(k, n)), gpu.zeros(Shape(m, n))
        gpu.fill_normal(x, SEED, 5000)
        gpu.fill_normal(w, SEED, 5001, 0.0, 0.02)
        spec = MatmulSpec.new(m, n, k)
        entry = {}
        for name, s in (("fp32", spec), ("bf16", spec.with_precision(Precision.Bf16))):
            ms = reference_method_ms(events, gpu.stream, lambda: gpu.matmul(s, x, w, y))
            entry[f"gflops_{name}"] = round(s.flops() / (ms * 1e-3) / 1e9, 1)
            entry[f"us_{name}"] = round(ms * 1e3, 2)
        entry["reference_orin_nx_blocked_gflops"] = orin
        entry["reference_agx_thor_tf32_gflops"] = thor
        result["products"][f"{label} {m}x{n}x{k} NN"] = entry
        for t in (x, w, y):
            t.free()
    for model, key in ((MODEL_7M, "config0_7.1M_set"), (MODEL_43M, "config1_42.9M_set")):
        calls, buffers = build_set(gpu, model)
        flops = sum(spec.flops() for _, _, spec, _ in calls)
        ms, per_call = measure_set(gpu, events, calls, 3, 1)
        _, per_layout, per_shape = summarize_set(calls, per_call, PEAK_FP32_TFLOPS)
        replay_ms = replayed_step_ms(gpu, events, calls, 5)
        result[key] = {"tflops": round(flops / (ms * 1e-3) / 1e12, 2), "ms_per_step": round(ms, 3),
                       "frac_fp32_peak": round(flops / (ms * 1e-3) / 1e12 / PEAK_FP32_TFLOPS, 4),
                       "graph_replay": {"tflops": round(flops / (replay_ms * 1e-3) / 1e12, 2),
                                        "ms_per_step": round(replay_ms, 3),
                                        "frac_fp32_peak": round(flops / (replay_ms * 1e-3) / 1e12 / PEAK_FP32_TFLOPS,
                                                                4)},
                       "gemms": len(calls), "tflop": round(flops / 1e12, 4), "per_layout": per_layout,
                       "per_shape_tflops": per_shape}
        for buf in buffers:
            for t in (buf.x, buf.w, buf.dy, buf.y, buf.dx, buf.dw):
                t.free()
    result["config2_weakest"] = {k: {"tflops": v, "frac_fp32_peak": round(v / PEAK_FP32_TFLOPS, 4)}
                                 for k, v in sorted(set_per_shape.items(), key=lambda kv: kv[1])[:2]}
    return result


# ---- one GPU's share of config 2 sharded over 8 GPUs -----------------------------------

def measure_shard_share(gpu: Gpu, events: HipEvents, shards: int = 8):
    """Config 2's set at the shape one GPU runs when the tokens are split over `shards` GPUs (the
    Linear products shard along M with no exchange; the weight gradients then sum over the shards,
    which this one-GPU run does not do): M = 32768 / shards, weight-gradient K the same."""
    model = dict(MODEL_111M, name=f"111.5M / {shards}", tokens=MODEL_111M["tokens"] // shards)
    calls, buffers = build_set(gpu, model)
    flops = sum(spec.flops() for _, _, spec, _ in calls)
    ms, per_call = measure_set(gpu, events, calls, 3, 1)
    _, per_layout, per_shape = summarize_set(calls, per_call, PEAK_FP32_TFLOPS)
    replay_ms = replayed_step_ms(gpu, events, calls, 3)
    for buf in buffers:
        for t in (buf.x, buf.w, buf.dy, buf.y, buf.dx, buf.dw):
            t.free()
    return {"shards": shards, "per_shape_tflops": per_shape, "tokens": model["tokens"], "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
            "frac_fp32_peak": round(flops / (ms * 1e-3) / 1e12 / PEAK_FP32_TFLOPS, 4),
            "ms_per_step": round(ms, 3), "per_layout": per_layout,
            "graph_replay": {"tflops": round(flops / (replay_ms * 1e-3) / 1e12, 2), "ms_per_step": round(replay_ms, 3),
                             "frac_fp32_peak": round(flops / (replay_ms * 1e-3) / 1e12 / PEAK_FP32_TFLOPS, 4)}}


# ---- the vendor library on the same set, and the clock under load (context) -------------

def _sclk_mhz():
    """The shader clock rocm-smi reports now, or None where the tool is absent."""
    try:
        text = subprocess.run(["rocm-smi", "--showclocks"], capture_output=True, text=True, timeout=10).stdout
    except (OSError, subprocess.SubprocessError):
        return None
    for line in text.splitlines():
        if "sclk" in line and "Mhz" in line:
            return int(line.rsplit("(", 1)[1].split("Mhz")[0])
    return None


def clocks_under_load(gpu: Gpu, calls, precision, seconds: float = 4.0):
    """Steps of the set run back to back for `seconds` while the shader clock is sampled."""
    import threading
    samples, stop = [], threading.Event()

    def sample():
        while not stop.is_set():
            mhz = _sclk_mhz()
            if mhz is not None:
                samples.append(mhz)
            time.sleep(0.3)

    run_step(gpu, calls, precision)
    gpu.synchronize()
    thread = threading.Thread(target=sample)
    thread.start()
    start, steps = time.time(), 0
    while time.time() - start < seconds:
        run_step(gpu, calls, precision)
        gpu.synchronize()
        steps += 1
    stop.set()
    thread.join()
    steady = samples[2:] or samples
    return {"steps": steps, "sclk_mhz_median": int(np.median(steady)) if steady else None,
            "samples": len(samples)}


def measure_vendor(gpu: Gpu, events: HipEvents, calls, repeats: int = 5):
    """Config 2's set through torch.mm (hipBLASLt / rocBLAS) on the same shapes and layouts: fp32
    (TF32 off); bf16 with the fp32 operands rounded inside the timed call, as this build's bf16
    contract does; and bf16 with the operands already bf16 in HBM (half the bytes, bf16 output).
    Each of the 15 distinct products is timed on torch's stream and weighted by its count in the
    set. Beside it, this build's own set in the same process, and the shader clock during each."""
    import torch
    torch.backends.cuda.matmul.allow_tf32 = False
    dev = torch.device("cuda", 0)

    def ms_of(fn):
        fn()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(repeats):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / repeats

    counts = {}
    for label, _, _, _ in calls[::3]:
        name = label.split(".")[-1]
        counts[name] = counts.get(name, 0) + 1
    d, f, heads, m = MODEL_111M["width"], MODEL_111M["ffn"], MODEL_111M["heads_width"], MODEL_111M["tokens"]
    layers = {"qkv": (d, 3 * d), "out": (d, d), "up": (d, f), "down": (f, d), "head": (d, heads)}
    per_shape, totals, set_flops = {}, {"f32": 0.0, "bf16_from_f32": 0.0, "bf16_inputs": 0.0}, 0.0
    gen = torch.Generator(device=dev).manual_seed(SEED)
    for name, (i, o) in layers.items():
        x = torch.randn(m, i, device=dev, generator=gen)
        w = torch.randn(i, o, device=dev, generator=gen) * 0.02
        dy = torch.randn(m, o, device=dev, generator=gen)
        y, dx, dw = torch.empty(m, o, device=dev), torch.empty(m, i, device=dev), torch.zeros(i, o, device=dev)
        xb, wb, dyb, dwb = x.bfloat16(), w.bfloat16(), dy.bfloat16(), dw.bfloat16()
        # Two-dimensional products only (no batched bf16 calls).
        variants = {
            "NN": (lambda: torch.mm(x, w, out=y), lambda: torch.mm(x.bfloat16(), w.bfloat16()).float(),
                   lambda: torch.mm(xb, wb), (m, o, i)),
            "TN": (lambda: dw.addmm_(x.t(), dy), lambda: dw.add_(torch.mm(x.bfloat16().t(), dy.bfloat16()).float()),
                   lambda: dwb.addmm_(xb.t(), dyb), (i, o, m)),
            "NT": (lambda: torch.mm(dy, w.t(), out=dx), lambda: torch.mm(dy.bfloat16(), w.bfloat16().t()).float(),
                   lambda: torch.mm(dyb, wb.t()), (m, i, o)),
        }
        flops = 2.0 * m * i * o
        for layout, (f32, from_f32, inputs, (r, c, k)) in variants.items():
            t = {"f32": ms_of(f32), "bf16_from_f32": ms_of(from_f32), "bf16_inputs": ms_of(inputs)}
            per_shape[f"{layout} {r}x{c}x{k}"] = {key: round(flops / (v * 1e-3) / 1e12, 1) for key, v in t.items()}
            for key, v in t.items():
                totals[key] += v * counts[name]
            set_flops += flops * counts[name]
        del x, w, dy, y, dx, dw, xb, wb, dyb, dwb
        torch.cuda.empty_cache()

    # One decode token (M = 1, 49 distinct weights, 390 MB > the Infinity Cache) through torch.mm,
    # captured in one graph as this build's token is, checked against the same calls run eagerly.
    layers = [(k, n) for _ in range(12) for _, k, n in DECODE_SHAPES[:4]] + [DECODE_SHAPES[4][1:]]
    token = [(torch.randn(1, k, device=dev, generator=gen), torch.randn(k, n, device=dev, generator=gen) * 0.02,
              torch.empty(1, n, device=dev)) for k, n in layers]
    for x, w, y in token:
        torch.mm(x, w, out=y)
    eager = [y.clone() for _, _, y in token]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for x, w, y in token:
            torch.mm(x, w, out=y)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for x, w, y in token:
            torch.mm(x, w, out=y)
    token_ms = ms_of(graph.replay)
    replay_matches = all(torch.equal(e, y) for e, (_, _, y) in zip(eager, token))
    token_bytes = sum(decode_bytes(1, k, n) for k, n in layers)
    del graph, token, eager
    torch.cuda.empty_cache()

    own_ms, _ = measure_set(gpu, events, calls, 3, 1)
    own_bf16_ms, _ = measure_set(gpu, events, calls, 3, 1, Precision.Bf16)
    return {
        "decode_token": {"us_per_token": round(token_ms * 1e3, 1), "gbs": round(token_bytes / (token_ms * 1e-3) / 1e9, 1),
                         "replay_matches_eager": replay_matches,
                         "method": "49 torch.mm (M = 1) captured in one graph, mean of replays"},
        "library": f"torch {torch.__version__} (HIP {torch.version.hip}) torch.mm / addmm_",
        "method": f"mean of {repeats} calls after 1 warm-up per product, weighted by the product's count in the set",
        "set_tflops": {key: round(set_flops / (v * 1e-3) / 1e12, 1) for key, v in totals.items()},
        "this_build_set_tflops": {"f32": round(set_flops / (own_ms * 1e-3) / 1e12, 1),
                                  "bf16": round(set_flops / (own_bf16_ms * 1e-3) / 1e12, 1)},
        "per_shape_tflops": per_shape,
        "clocks": {"f32_set": clocks_under_load(gpu, calls, Precision.Default),
                   "bf16_set": clocks_under_load(gpu, calls, Precision.Bf16),
                   "idle_sclk_mhz": _sclk_mhz()},
    }


# ---- Linear's bias kernels (the steps either side of the NN and TN products) -----------

def measure_linear(gpu: Gpu, events: HipEvents, buffers, repeats: int = 5):
    """Config 2's Linear layers (block 0's four and the head): the forward as the reference
    calls it (matmul, then add_row_bias; linear.rs:46-47) against the fused sn_matmul_bias, and
    the bias gradient (accumulate_column_sums, linear.rs:59), with the bias kernels' HBM rates
    (add_row_bias: 8 bytes per output element; column sums: 4 bytes per input element); and the
    weight and bias gradients as the reference calls them (matmul, then accumulate_column_sums;
    linear.rs:54-59) against sn_matmul_column_sums, the sums taken inside the product; forward and
    gradients in fp32 and at bf16 precision."""
    layers = [b for b, (label, _, _) in zip(buffers, training_set()) if label.startswith("b0.") or label == "head"]
    names = ["qkv", "out", "up", "down", "head"]
    result = {}
    for name, buf in zip(names, layers):
        m, n = buf.y.shape().rows, buf.y.shape().cols
        k = buf.x.shape().cols
        bias = gpu.zeros(Shape.vector(n))
        gpu.fill_normal(bias, SEED, 4000, 0.0, 0.02)
        sums = gpu.zeros(Shape.vector(n))
        spec = MatmulSpec.new(m, n, k)
        gpu.matmul(spec, buf.x, buf.w, buf.y)  # warm-up of each call
        gpu.add_row_bias(buf.y, bias)
        gpu.matmul_bias(spec, buf.x, buf.w, bias, buf.y)
        gpu.accumulate_column_sums(buf.dy, sums)
        separate = timed(events, gpu.stream, lambda: (gpu.matmul(spec, buf.x, buf.w, buf.y),
                                                       gpu.add_row_bias(buf.y, bias)), repeats)
        fused = timed(events, gpu.stream, lambda: gpu.matmul_bias(spec, buf.x, buf.w, bias, buf.y), repeats)
        bias_ms = timed(events, gpu.stream, lambda: gpu.add_row_bias(buf.y, bias), repeats)
        sums_ms = timed(events, gpu.stream, lambda: gpu.accumulate_column_sums(buf.dy, sums), repeats)
        grad = MatmulSpec.new(k, n, m).left_transposed().accumulate()
        gpu.matmul_column_sums(grad, buf.x, buf.dy, buf.dw, sums)
        grads_separate = timed(events, gpu.stream, lambda: (gpu.matmul(grad, buf.x, buf.dy, buf.dw),
                                                             gpu.accumulate_column_sums(buf.dy, sums)), repeats)
        grads_fused = timed(events, gpu.stream, lambda: gpu.matmul_column_sums(grad, buf.x, buf.dy, buf.dw, sums),
                            repeats)
        spec16 = spec.with_precision(Precision.Bf16)
        gpu.matmul_bias(spec16, buf.x, buf.w, bias, buf.y)
        separate16 = timed(events, gpu.stream, lambda: (gpu.matmul(spec16, buf.x, buf.w, buf.y),
                                                         gpu.add_row_bias(buf.y, bias)), repeats)
        fused16 = timed(events, gpu.stream, lambda: gpu.matmul_bias(spec16, buf.x, buf.w, bias, buf.y), repeats)
        grad16 = grad.with_precision(Precision.Bf16)
        gpu.matmul_column_sums(grad16, buf.x, buf.dy, buf.dw, sums)
        grads16_separate = timed(events, gpu.stream, lambda: (gpu.matmul(grad16, buf.x, buf.dy, buf.dw),
                                                               gpu.accumulate_column_sums(buf.dy, sums)), repeats)
        grads16_fused = timed(events, gpu.stream,
                              lambda: gpu.matmul_column_sums(grad16, buf.x, buf.dy, buf.dw, sums), repeats)
        result[f"{name} {m}x{n}x{k}"] = {
            "forward_separate_ms": round(separate, 4), "forward_fused_ms": round(fused, 4),
            "fused_saving_pct": round(100 * (1 - fused / separate), 1),
            "add_row_bias_gbs": round(8 * m * n / (bias_ms * 1e-3) / 1e9, 1),
            "column_sums_ms": round(sums_ms, 4),
            "column_sums_gbs": round(4 * m * n / (sums_ms * 1e-3) / 1e9, 1),
            "weight_bias_grads_separate_ms": round(grads_separate, 4),
            "weight_bias_grads_fused_ms": round(grads_fused, 4),
            "grads_fused_saving_pct": round(100 * (1 - grads_fused / grads_separate), 1),
            "bf16_forward_separate_ms": round(separate16, 4), "bf16_forward_fused_ms": round(fused16, 4),
            "bf16_fused_saving_pct": round(100 * (1 - fused16 / separate16), 1),
            "bf16_weight_bias_grads_separate_ms": round(grads16_separate, 4),
            "bf16_weight_bias_grads_fused_ms": round(grads16_fused, 4),
            "bf16_grads_fused_saving_pct": round(100 * (1 - grads16_fused / grads16_separate), 1)}
        bias.free()
        sums.free()
    return result


def measure_loss(gpu: Gpu, events: HipEvents, buffers, repeats: int = 3):
    """The head product's consumer at config 2 (training.rs:208-239): softmax cross-entropy and its
    gradient for each of the 16 codebooks over the [32768, 16 x 1024] logits, one call per codebook
    as the reference makes them. HBM rate on 8 bytes per logit (read the logits, write the gradient)."""
    from staleynet_amd.gemm import CrossEntropyHead
    head = buffers[-1]
    rows, cols = head.y.shape().rows, head.y.shape().cols
    codebooks, size = 16, cols // 16
    rng = np.random.default_rng(SEED)
    targets = gpu.upload_tokens(rng.integers(0, size, rows * codebooks).astype(np.uint32))
    losses, grad = gpu.zeros(Shape.vector(rows)), gpu.zeros(Shape(rows, cols))
    heads = [CrossEntropyHead(c * size, size, codebooks, c, 1.0 / (rows * codebooks)) for c in range(codebooks)]

    def all_codebooks():
        for h in heads:
            gpu.cross_entropy(head.y, targets, h, losses, grad)

    all_codebooks()
    ms = timed(events, gpu.stream, all_codebooks, repeats)
    grad.free()
    losses.free()
    targets.free()
    return {"codebooks": codebooks, "shape": f"{rows}x{cols}", "ms_all_codebooks": round(ms, 3),
            "gbs": round(8 * rows * cols / (ms * 1e-3) / 1e9, 1)}


# ---- CPU baseline -----------------------------------------------------------------------

def cpu_baseline(gpu: Gpu, calls, budget_s: float, workers: int = 1):
    """Times the oracle (reference::matmul restated in C) on a row sample of
    each distinct GEMM of the set, using the GPU's own input bytes, and scales
    each to its full size (cost is linear in output rows). One core, or with
    workers > 1 the sample's rows split across that many threads (each element
    still computed exactly as in the serial loop)."""
    from concurrent.futures import ThreadPoolExecutor

    from oracle import oracle

    pool = ThreadPoolExecutor(workers) if workers > 1 else None

    def run_rows(product, a, b, c, first, count):
        if pool is None:
            oracle.matmul_rows(product, a, b, c, first, first + count)
            return
        bounds = [first + count * i // workers for i in range(workers + 1)]
        list(pool.map(lambda i: oracle.matmul_rows(product, a, b, c, bounds[i], bounds[i + 1]), range(workers)))

    distinct = {}
    for label, layout, spec, ops in calls:
        key = (layout, spec.rows, spec.cols, spec.inner)
        distinct.setdefault(key, [spec, ops, 0])
        distinct[key][2] += 1
    per_gemm_budget = budget_s / len(distinct)
    projected_s, sampled_flops, sampled_s, samples = 0.0, 0, 0.0, []
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
        n_rows = int(max(1, min(rows - 1, workers * per_gemm_budget / one_row)))
        t0 = time.perf_counter()
        run_rows(product, a, b, c, 1, n_rows)
        elapsed = time.perf_counter() - t0
        rate = 2.0 * n_rows * cols * inner / elapsed
        projected_s += count * spec.flops() / rate
        sampled_flops += 2 * n_rows * cols * inner
        sampled_s += elapsed
        samples.append(f"{layout} {rows}x{cols}x{inner}: {n_rows} rows")
        del a, b, c
    if pool is not None:
        pool.shutdown()
    return projected_s, sampled_flops, sampled_s, samples


def parse_rocminfo_gpu(text: str):
    """(compute units, max engine clock in MHz) of the first gfx9 GPU agent in `rocminfo` output,
    or None when no such agent is listed."""
    agent = None
    for line in text.splitlines():
        key, _, value = line.strip().partition(":")
        key, value = key.strip(), value.strip()
        if key == "Name":
            if agent and agent.get("gpu") and "cus" in agent and "mhz" in agent:
                break
            agent = {"gpu": value.startswith("gfx9")}
        elif agent is not None and agent["gpu"]:
            if key == "Compute Unit" and value.isdigit():
                agent["cus"] = int(value)
            elif key == "Max Clock Freq. (MHz)" and value.isdigit():
                agent["mhz"] = int(value)
    if agent and agent.get("gpu") and "cus" in agent and "mhz" in agent:
        return agent["cus"], agent["mhz"]
    return None


def device_peaks() -> dict:
    """The peaks recomputed from the device's own compute-unit count and maximum engine clock
    (rocminfo), beside the published figures the fractions use: fp32 matrix 256 FLOP per clock
    per CU, bf16 dense 4096."""
    try:
        text = subprocess.run([os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "rocminfo")],
                              stdout=subprocess.PIPE, stderr=subprocess.DEVNULL, text=True, timeout=60).stdout
    except (OSError, subprocess.SubprocessError):
        return {"source": "rocminfo unavailable"}
    found = parse_rocminfo_gpu(text)
    if found is None:
        return {"source": "rocminfo lists no gfx9 GPU agent"}
    cus, mhz = found
    return {"source": "rocminfo", "compute_units": cus, "max_engine_clock_mhz": mhz,
            "fp32_matrix_tflops_from_clock": round(cus * 256 * mhz * 1e6 / 1e12, 1),
            "bf16_dense_tflops_from_clock": round(cus * 4096 * mhz * 1e6 / 1e12, 1),
            "published_fp32_tflops": PEAK_FP32_TFLOPS, "published_bf16_tflops": PEAK_BF16_TFLOPS,
            "published_hbm_gbs": PEAK_HBM_GBS}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


# ---- rocprofv3 summaries ----------------------------------------------------------------

# The roofline kernel: the persistent direct-to-LDS fp32 MFMA kernel, 128x128 tile, A K-contiguous, B
# N-contiguous (every forward NN product of config 2's set).
NN_KERNEL_KEY = ("gemm_f32_persistent_kernel<sn::gemm::(anonymous namespace)::DmaConfig<sn::gemm::Tile<128, 128, 32, "
                 "2, 2>, 2>, true, false>")
COPY_KERNEL_KEY = "copy_kernel("
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "gemm_f32_nn_111M_hbm_traffic.txt")


def load_traffic(path: str = TRAFFIC_SUMMARY):
    """HBM bytes per NN launch from the committed PMC summary, or None without one."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def _short(name: str) -> str:
    name = name.replace("sn::gemm::", "").replace("(anonymous namespace)::", "").replace("sn::", "")
    return name.split("(")[0] if "(" in name else name


def _per_dispatch(csv_path: str, counter: str):
    """{kernel name: [counter value per dispatch, in dispatch order]} from a counter_collection.csv."""
    import csv
    out = {}
    with open(csv_path, newline="") as f:
        rows = sorted((r for r in csv.DictReader(f) if r["Counter_Name"] == counter),
                      key=lambda r: int(r["Dispatch_Id"]))
    for r in rows:
        out.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
    return out


def summarize_pmc(fetch_csv: str, write_csv: str, copy_mib: int) -> str:
    """HBM traffic of the NN kernel per launch: FETCH_SIZE and WRITE_SIZE (KiB per dispatch), each
    divided by what the same counter reads for the plain copy kernel per byte it moves."""
    fetch, write = _per_dispatch(fetch_csv, "FETCH_SIZE"), _per_dispatch(write_csv, "WRITE_SIZE")
    pick = lambda table, key: next(v for k, v in table.items() if key in k)  # noqa: E731
    copy_bytes = copy_mib << 20
    f_copy, w_copy = pick(fetch, COPY_KERNEL_KEY), pick(write, COPY_KERNEL_KEY)
    f_factor = f_copy[-1] * 1024 / copy_bytes
    w_factor = w_copy[-1] * 1024 / copy_bytes
    f_nn, w_nn = pick(fetch, NN_KERNEL_KEY), pick(write, NN_KERNEL_KEY)
    nn_calls = [spec for _, layout, spec in _set_specs() if layout == "NN"]
    assert len(f_nn) == len(w_nn) == len(nn_calls), (len(f_nn), len(w_nn), len(nn_calls))
    lines = [f"copy kernel ({copy_mib} MiB read + {copy_mib} MiB written): FETCH_SIZE {f_copy[-1]:.0f} KiB, "
             f"WRITE_SIZE {w_copy[-1]:.0f} KiB -> factors {f_factor:.4f} (fetch), {w_factor:.4f} (write)",
             "", "NN launches of one step, grouped by shape (means per launch):",
             f"{'shape MxNxK':>22} {'launches':>8} {'algorithmic MB':>15} {'HBM read MB':>12} {'HBM write MB':>13} "
             f"{'traffic/alg':>11}"]
    groups = {}
    for spec, f, w in zip(nn_calls, f_nn, w_nn):
        g = groups.setdefault((spec.rows, spec.cols, spec.inner), [0, 0.0, 0.0])
        g[0] += 1
        g[1] += f * 1024 / f_factor
        g[2] += w * 1024 / w_factor
    for (m, n, k), (count, rd, wr) in groups.items():
        alg = 4 * (m * k + k * n + m * n)
        lines.append(f"{f'{m}x{n}x{k}':>22} {count:>8} {alg / 1e6:>15.1f} {rd / count / 1e6:>12.1f} "
                     f"{wr / count / 1e6:>13.1f} {(rd + wr) / count / alg:>11.3f}")
    traffic = sum(f * 1024 / f_factor + w * 1024 / w_factor for f, w in zip(f_nn, w_nn)) / len(f_nn)
    algorithmic = sum(4 * (s.rows * s.inner + s.inner * s.cols + s.rows * s.cols) for s in nn_calls) / len(nn_calls)
    lines += ["", f"raw counter means per NN launch: FETCH_SIZE {sum(f_nn) / len(f_nn):.0f} KiB, "
              f"WRITE_SIZE {sum(w_nn) / len(w_nn):.0f} KiB",
              f"mean over the {len(nn_calls)} NN launches: algorithmic {algorithmic / 1e6:.1f} MB, "
              f"HBM traffic {traffic / 1e6:.1f} MB ({traffic / algorithmic:.3f}x)",
              f"traffic_bytes_per_launch: {int(round(traffic))}",
              f"algorithmic_bytes_per_launch: {int(round(algorithmic))}"]
    return "\n".join(lines)


GEMV_KERNEL_KEY = "gemv_kernel<"


def _in_dispatch_order(csv_path: str, counter: str, key: str):
    """Values of `counter` for every dispatch whose kernel name holds `key` (the GEMV's name
    differs per row count), in dispatch order, from a counter_collection.csv."""
    import csv
    with open(csv_path, newline="") as f:
        rows = sorted((r for r in csv.DictReader(f) if r["Counter_Name"] == counter and key in r["Kernel_Name"]),
                      key=lambda r: int(r["Dispatch_Id"]))
    return [float(r["Counter_Value"]) for r in rows]


def _trace_durations(trace_csv: str, key: str):
    """Durations (ns) of the dispatches whose kernel name holds `key`, in dispatch order, from a
    rocprofv3 kernel_trace.csv."""
    import csv
    with open(trace_csv, newline="") as f:
        rows = sorted((r for r in csv.DictReader(f) if key in r["Kernel_Name"]), key=lambda r: int(r["Dispatch_Id"]))
    return [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in rows]


def summarize_decode_pmc(fetch_csv: str, write_csv: str, trace_csv: str, copy_mib: int) -> str:
    """HBM bytes and GB/s of the decode GEMV per shape: FETCH_SIZE and WRITE_SIZE per dispatch
    (copy-calibrated as in summarize_pmc) over the kernel's duration from a separate kernel-trace
    run of the same workload; the measured dispatches of each shape only."""
    fetch, write = _per_dispatch(fetch_csv, "FETCH_SIZE"), _per_dispatch(write_csv, "WRITE_SIZE")
    copy_bytes = copy_mib << 20
    pick = lambda table, key: next(v for k, v in table.items() if key in k)  # noqa: E731
    f_factor = pick(fetch, COPY_KERNEL_KEY)[-1] * 1024 / copy_bytes
    w_factor = pick(write, COPY_KERNEL_KEY)[-1] * 1024 / copy_bytes
    f_gemv = _in_dispatch_order(fetch_csv, "FETCH_SIZE", GEMV_KERNEL_KEY)
    w_gemv = _in_dispatch_order(write_csv, "WRITE_SIZE", GEMV_KERNEL_KEY)
    durations = _trace_durations(trace_csv, GEMV_KERNEL_KEY)
    launches = list(_decode_pmc_launches())
    assert len(f_gemv) == len(w_gemv) == len(durations) == len(launches), \
        (len(f_gemv), len(w_gemv), len(durations), len(launches))
    groups = {}
    for (m, name, k, n, _, measured), f, w, ns in zip(launches, f_gemv, w_gemv, durations):
        if measured:
            g = groups.setdefault((m, name, k, n), [0, 0.0, 0.0, 0.0])
            g[0] += 1
            g[1] += f * 1024 / f_factor
            g[2] += w * 1024 / w_factor
            g[3] += ns
    lines = [f"copy kernel ({copy_mib} MiB read + {copy_mib} MiB written): factors {f_factor:.4f} (fetch), "
             f"{w_factor:.4f} (write)", "",
             f"{'product':>24} {'alg MB':>8} {'HBM rd MB':>10} {'HBM wr MB':>10} {'traffic/alg':>11} "
             f"{'kernel us':>10} {'alg GB/s':>9} {'HBM GB/s':>9} {'of 8 TB/s':>9}"]
    for (m, name, k, n), (count, rd, wr, ns) in groups.items():
        alg = decode_bytes(m, k, n)
        rd, wr, ns = rd / count, wr / count, ns / count
        lines.append(f"{f'M={m} {name} {k}x{n}':>24} {alg / 1e6:>8.2f} {rd / 1e6:>10.2f} {wr / 1e6:>10.3f} "
                     f"{(rd + wr) / alg:>11.3f} {ns / 1e3:>10.2f} {alg / ns:>9.0f} {(rd + wr) / ns:>9.0f} "
                     f"{(rd + wr) / ns / PEAK_HBM_GBS:>9.3f}")
    return "\n".join(lines)


def summarize_counters(csv_paths) -> str:
    """Per-kernel means over dispatches of every counter in one or more rocprofv3
    counter_collection.csv files (one counter group per run), with the derived shares:
    MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (4 SIMDs x SQ_BUSY_CU_CYCLES); waiting =
    SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES; VALU per MFMA = (SQ_INSTS_VALU - SQ_INSTS_MFMA) / SQ_INSTS_MFMA."""
    import csv
    sums = {}
    for path in csv_paths:
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                k = sums.setdefault(_short(r["Kernel_Name"]), {}).setdefault(r["Counter_Name"], [0.0, 0])
                k[0] += float(r["Counter_Value"])
                k[1] += 1
    lines = []
    for kernel, counters in sums.items():
        mean = {name: total / count for name, (total, count) in counters.items()}
        derived = []
        if "SQ_VALU_MFMA_BUSY_CYCLES" in mean and mean.get("SQ_BUSY_CU_CYCLES"):
            derived.append(f"MFMA busy {mean['SQ_VALU_MFMA_BUSY_CYCLES'] / (4 * mean['SQ_BUSY_CU_CYCLES']):.3f}")
        if "SQ_WAIT_INST_ANY" in mean and mean.get("SQ_WAVE_CYCLES"):
            derived.append(f"waiting {mean['SQ_WAIT_INST_ANY'] / mean['SQ_WAVE_CYCLES']:.3f}")
        if mean.get("SQ_INSTS_MFMA") and "SQ_INSTS_VALU" in mean:
            derived.append(f"VALU per MFMA {(mean['SQ_INSTS_VALU'] - mean['SQ_INSTS_MFMA']) / mean['SQ_INSTS_MFMA']:.2f}")
        lines.append(f"{kernel[:90]}")
        if derived:
            lines.append("    " + "; ".join(derived))
        for name in sorted(mean):
            lines.append(f"    {name:<28} {mean[name]:>16.0f}")
    return "\n".join(lines)


def summarize_trace(stats_csv: str, bench_json: str = "") -> str:
    """Kernel table from rocprofv3's kernel_stats.csv; with the bench line of the same run, the NN
    kernel's rocprof average beside the HIP-event mean bench.py reported."""
    import csv
    with open(stats_csv, newline="") as f:
        rows = list(csv.DictReader(f))
    lines = [f"{'kernel':<92} {'calls':>6} {'avg us':>9} {'min us':>9} {'max us':>9} {'total ms':>9} {'%':>6}"]
    for r in rows:
        lines.append(f"{_short(r['Name'])[:92]:<92} {int(r['Calls']):>6} {float(r['AverageNs']) / 1e3:>9.1f} "
                     f"{float(r['MinNs']) / 1e3:>9.1f} {float(r['MaxNs']) / 1e3:>9.1f} "
                     f"{float(r['TotalDurationNs']) / 1e6:>9.2f} {float(r['Percentage']):>6.2f}")
    nn = next((r for r in rows if NN_KERNEL_KEY in r["Name"]), None)
    if nn is not None and bench_json:
        with open(bench_json) as f:
            line = json.loads([x for x in f.read().splitlines() if x.startswith("{")][-1])
        event_ms = line["roofline"]["launch_ms_mean"]
        prof_ms = float(nn["AverageNs"]) / 1e6
        lines += ["", f"NN roofline kernel: rocprof average {prof_ms:.4f} ms over {nn['Calls']} launches; "
                  f"bench.py HIP-event mean {event_ms:.4f} ms (ratio {event_ms / prof_ms:.3f})"]
    return "\n".join(lines)


def _set_specs():
    """(label, layout, spec) of every product of the set, in launch order, without a GPU."""
    model = MODEL_111M
    for label, inputs, outputs in training_set(model):
        for layout, spec in linear_products(model["tokens"], inputs, outputs):
            yield label, layout, spec


# ---- main -------------------------------------------------------------------------------

def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=5)
    parser.add_argument("--warmup", type=int, default=1)
    parser.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU-baseline sampling")
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    parser.add_argument("--no-extras", action="store_true", help="only the fp32 set (bf16, attention, decode off)")
    parser.add_argument("--copy-calibration-mib", type=int, default=0,
                        help="run one plain copy of this many MiB first (the PMC byte-counter calibration)")
    parser.add_argument("--summarize-trace", nargs="+", metavar=("KERNEL_STATS_CSV", "BENCH_JSON"),
                        help="print a kernel table from a rocprofv3 --stats run and exit (no GPU)")
    parser.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                        help="print the NN kernel's HBM traffic from two --pmc runs and exit (no GPU)")
    parser.add_argument("--summarize-counters", nargs="+", metavar="COUNTER_CSV",
                        help="print per-kernel counter means (and MFMA busy, wait share) from rocprofv3 --pmc "
                             "counter_collection.csv files and exit (no GPU)")
    parser.add_argument("--decode-pmc", action="store_true",
                        help="run only the decode counter workload (each config-4 product over a weight pool, "
                             "plain launches; with --copy-calibration-mib, the calibration copy first) and exit")
    parser.add_argument("--summarize-decode-pmc", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "KERNEL_TRACE_CSV"),
                        help="print the decode GEMV's HBM bytes and GB/s per product from two --pmc runs and a "
                             "kernel-trace run of --decode-pmc, and exit (no GPU)")
    parser.add_argument("--decode-attention-pmc", action="store_true",
                        help="run only the decode-attention counter workload (the fused decode form, then the "
                             "reference's three calls, over a pool of caches; with --copy-calibration-mib, the "
                             "calibration copy first) and exit")
    parser.add_argument("--summarize-kernel-pmc", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "KERNEL_TRACE_CSV"),
                        help="print HBM bytes and durations per decode-attention kernel from two --pmc runs and a "
                             "kernel-trace run of --decode-attention-pmc, and exit (no GPU)")
    parser.add_argument("--one-attention", choices=["forward", "forward_p", "score_grad", "score_grad_dq",
                                                    "forward_stats", "backward"],
                        help="run only config 3's fused attention kernel 1 + 5 times and exit: the workload of the "
                             "attention counter profiles")
    parser.add_argument("--plain-launches", action="store_true",
                        help="replay the decode measurements' launches directly instead of from HIP graphs (for "
                             "profiled runs: the timings then include host launch costs)")
    parser.add_argument("--one-product", nargs=2, metavar=("LAYOUT", "PRECISION"),
                        help="run only config 2's qkv product (NN, TN or NT; f32 or bf16) 1 + 5 times and exit: "
                             "the workload of the per-kernel counter profiles")
    parser.add_argument("--vendor", action="store_true",
                        help="run only the vendor-library comparison on config 2's set (torch.mm fp32 and bf16 "
                             "beside this build's set, and the shader clock under each set's load) and exit")
    parser.add_argument("--one-linear", action="store_true",
                        help="run only config 2's Linear bias measurements (block 0's four layers and the head: "
                             "forward with and without the fused bias, weight and bias gradients as two calls "
                             "and fused) and exit: the workload of the fused bias-gradient trace")
    args = parser.parse_args()

    if args.summarize_trace:
        print(summarize_trace(*args.summarize_trace[:2]))
        return 0
    if args.summarize_pmc:
        print(summarize_pmc(*args.summarize_pmc, args.copy_calibration_mib or 1024))
        return 0
    if args.summarize_counters:
        print(summarize_counters(args.summarize_counters))
        return 0
    if args.summarize_kernel_pmc:
        print(summarize_kernel_pmc(*args.summarize_kernel_pmc, args.copy_calibration_mib or 1024,
                                   decode_attention_algorithmic()))
        return 0
    if args.summarize_decode_pmc:
        print(summarize_decode_pmc(*args.summarize_decode_pmc, args.copy_calibration_mib or 1024))
        return 0

    if args.plain_launches:
        global REPLAY
        REPLAY = PlainReplay
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: the GEMM path runs on one device and its sharding is a design "
              f"note, not a measured path; got --gpus {args.gpus}", file=sys.stderr)
        return 2

    gpu = Gpu(0)
    events = HipEvents()
    if args.one_attention:
        print(json.dumps(run_one_attention(gpu, events, args.one_attention)))
        gpu.close()
        return 0
    if args.vendor:
        calls, _buffers = build_set(gpu)
        print(json.dumps({"vendor": measure_vendor(gpu, events, calls)}))
        gpu.close()
        return 0
    if args.one_linear:
        model = MODEL_111M
        buffers = [LinearBuffers(gpu, model["tokens"], inputs, outputs, 16 * index)
                   if label.startswith("b0.") or label == "head" else None
                   for index, (label, inputs, outputs) in enumerate(training_set(model))]
        gpu.synchronize()
        print(json.dumps({"linear_bias": measure_linear(gpu, events, buffers)}))
        gpu.close()
        return 0
    if args.one_product:
        layout, precision = args.one_product
        m, d = MODEL_111M["tokens"], MODEL_111M["width"]
        buf = LinearBuffers(gpu, m, d, 3 * d, 0)
        spec = dict(linear_products(m, d, 3 * d))[layout]
        if precision == "bf16":
            spec = spec.with_precision(Precision.Bf16)
        left, right, out = buf.operands(layout)
        ms = timed(events, gpu.stream, lambda: gpu.matmul(spec, left, right, out), 1)
        ms = timed(events, gpu.stream, lambda: gpu.matmul(spec, left, right, out), 5)
        print(json.dumps({"product": f"{layout} {spec.rows}x{spec.cols}x{spec.inner}", "precision": precision,
                          "ms": round(ms, 4), "tflops": round(spec.flops() / (ms * 1e-3) / 1e12, 1)}))
        gpu.close()
        return 0
    if args.copy_calibration_mib:
        src = gpu.zeros(Shape(args.copy_calibration_mib << 18, 1))
        dst = gpu.zeros(Shape(args.copy_calibration_mib << 18, 1))
        gpu.fill_normal(src, SEED, 3000)
        gpu.copy_device(dst, src)
        gpu.synchronize()
        src.free()
        dst.free()
    if args.decode_pmc:
        print(json.dumps({"decode_pmc_launches": run_decode_pmc_workload(gpu)}))
        gpu.close()
        return 0
    if args.decode_attention_pmc:
        print(json.dumps({"decode_attention_pmc_launches": run_decode_attention_pmc_workload(gpu)}))
        gpu.close()
        return 0
    calls, _buffers = build_set(gpu)
    set_flops = sum(spec.flops() for _, _, spec, _ in calls)

    ms_per_step, per_call = measure_set(gpu, events, calls, args.steps, args.warmup)
    layouts, per_layout, per_shape = summarize_set(calls, per_call, PEAK_FP32_TFLOPS)
    nn = layouts["NN"]
    nn_flops_per_launch = nn["flops"] / nn["launches"]
    nn_ms_per_launch = nn["ms"] / nn["launches"]
    achieved = nn_flops_per_launch / (nn_ms_per_launch * 1e-3) / 1e12
    roofline = {"kernel": "gemm_f32_persistent_kernel<DmaConfig<Tile<128,128,32,2,2>, 2 stages>, A K-contiguous, "
                          "B N-contiguous> (every forward NN product of the set)",
                "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP32_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / PEAK_FP32_TFLOPS, 4), "traffic": load_traffic(),
                "launch_ms_mean": round(nn_ms_per_launch, 4), "flops_per_launch": nn_flops_per_launch,
                "launches_per_step": nn["launches"],
                "traffic_unit": "HBM bytes per launch (PMC FETCH_SIZE + WRITE_SIZE, copy-calibrated; "
                                "profiles/gemm_f32_nn_111M_hbm_traffic.txt)",
                "algorithmic_bytes_per_launch": int(sum(4 * (s.rows * s.inner + s.inner * s.cols + s.rows * s.cols)
                                                        for _, y, s, _ in calls if y == "NN") / nn["launches"])}

    value = set_flops / (ms_per_step * 1e-3) / 1e12
    result = {
        "metric": METRIC,
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
        "device_peaks": device_peaks(),
        "roofline": roofline,
        "per_layout": per_layout,
        "per_shape_tflops": per_shape,
    }

    if not args.no_extras:
        bf16_steps = max(1, min(args.steps, 3))
        bf16_ms, bf16_calls = measure_set(gpu, events, calls, bf16_steps, 1, Precision.Bf16)
        bf16_tflops = set_flops / (bf16_ms * 1e-3) / 1e12
        attainable = set_flops / sum(spec.flops() / (bf16_roofline_tflops(spec) * 1e12) for _, _, spec, _ in calls) / 1e12
        _, bf16_layout, _ = summarize_set(calls, bf16_calls, PEAK_BF16_TFLOPS)
        result["bf16"] = {"value": round(bf16_tflops, 2), "unit": "TFLOP/s", "ms_per_step": round(bf16_ms, 3),
                          "frac_bf16_peak": round(bf16_tflops / PEAK_BF16_TFLOPS, 4),
                          "roofline_min_peak_or_ai_x_hbm": round(attainable, 1),
                          "frac_roofline": round(bf16_tflops / attainable, 4), "per_layout": bf16_layout,
                          "inputs": "fp32 in HBM; the 256x256 kernel rounds fp32 operand fragments to bf16 "
                                    "(nearest-even) as it loads them into LDS; an operand at most half the size "
                                    "of the other is first rounded into the context's workspace (timed with "
                                    "the product); bf16 matrix-core products with fp32 accumulation"}
        result["linear_bias"] = measure_linear(gpu, events, _buffers)
        result["head_cross_entropy"] = measure_loss(gpu, events, _buffers)
        result["attention"] = measure_attention(gpu, events)
        result["decode"] = measure_decode(gpu, events)
        result["published"] = measure_published(gpu, events, per_shape)
        result["shard_of_8"] = measure_shard_share(gpu, events)

    if not args.no_cpu:
        projected_s, sampled_flops, sampled_s, samples = cpu_baseline(gpu, calls, args.cpu_budget)
        result["cpu_baseline"] = {
            "value": round(set_flops / projected_s / 1e12, 8), "unit": "TFLOP/s", "cores": 1, "kind": "port",
            "sample": f"reference::matmul restated in C (oracle/), single thread, same input bytes; "
                      f"{sampled_flops / 1e9:.1f} GFLOP over row samples of the {len(samples)} distinct GEMMs "
                      f"({sampled_s:.1f} s), scaled linearly in rows to the full set: {projected_s:.0f} s per step",
            "host_cpu": _cpu_model(), "host_threads": os.cpu_count()}
        # The same loop with each sample's rows split across the host's cores (at most 16, the box's
        # share for one GPU), labelled as such: a reported variant, not the contract's baseline.
        workers = min(16, os.cpu_count() or 1)
        if workers > 1:
            projected_s, sampled_flops, sampled_s, samples = cpu_baseline(gpu, calls, args.cpu_budget / 4, workers)
            result["cpu_baseline_all_cores"] = {
                "value": round(set_flops / projected_s / 1e12, 8), "unit": "TFLOP/s", "cores": workers,
                "kind": "port",
                "sample": f"reference::matmul restated in C (oracle/), rows split over {workers} threads; "
                          f"{sampled_flops / 1e9:.1f} GFLOP over row samples of the {len(samples)} distinct GEMMs "
                          f"({sampled_s:.1f} s), scaled linearly in rows to the full set: {projected_s:.0f} s per step"}
    print(json.dumps(result))
    gpu.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
