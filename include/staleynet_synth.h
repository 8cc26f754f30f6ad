/*
 * staleynet_synth.h — seeded synthetic inputs for benchmarks and tests.
 *
 * No counterpart in the reference: its weights are drawn on the host
 * (crates/staleynet-model/src/random.rs) and its GEMM bench multiplies
 * zero-filled operands (crates/staleynet-cli/src/commands/bench.rs:131-138).
 * This generator fills device memory directly so that multi-gigabyte inputs
 * are resident in HBM before a timed region starts.
 */
#ifndef STALEYNET_SYNTH_H
#define STALEYNET_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Enqueues on `stream` (a hipStream_t, e.g. from sn_context_stream) a fill of
 * `count` floats at `device` with mean + std * N(0, 1) deviates: SplitMix64
 * counters + Box-Muller, keyed by (seed, stream_id). Returns 0, -1 for a null
 * buffer, or a HIP error code. */
int sn_fill_normal(void *stream, float *device, size_t count, uint64_t seed, uint64_t stream_id, float mean,
                   float stddev);

/* Enqueues on `stream` a copy of `count` floats from `src` to `dst` (both
 * device memory, 16-byte aligned, count a multiple of 4, not overlapping).
 * A plain streaming kernel used to calibrate hardware byte counters. Returns
 * 0, -1 for a null buffer, -7 for a misaligned buffer or count, or a HIP
 * error code. */
int sn_copy_device(void *stream, float *dst, const float *src, size_t count);

/* Enqueues on `stream` a streaming read of `count` floats at `src` (16-byte
 * aligned, count a multiple of 4) by `sums_count` workgroups (1..65535),
 * each writing the sum of its grid-stride share to sums[workgroup]. Measures
 * the practical HBM read bandwidth that read-bound kernels are compared
 * with. Returns 0, -1 for a null buffer, -7 for a misaligned buffer or bad
 * count, or a HIP error code. */
int sn_read_sum(void *stream, const float *src, size_t count, float *sums, size_t sums_count);

#ifdef __cplusplus
}
#endif

#endif /* STALEYNET_SYNTH_H */
